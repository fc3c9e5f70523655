// zcgvs_engine: the reference's Python module (bindings/python/module.cpp:18-192) over this build's
// Engine, plus the vector-query entry points (search_vectors, retrieve_vectors, add_vectors), a
// subclassable QueryEmbedder for text queries, and the artifact classes for tools and tests.
// Blocking calls release the GIL; the Engine serializes them itself.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <memory>
#include <string>
#include <vector>

#include "zcgvs/data/corpus.hpp"
#include "zcgvs/data/embedding_store.hpp"
#include "zcgvs/data/lexical_index.hpp"
#include "zcgvs/engine/engine.hpp"

namespace py = pybind11;

namespace {

using FloatRows = py::array_t<float, py::array::c_style | py::array::forcecast>;

class PyQueryEmbedder : public zcgvs::QueryEmbedder {
public:
    std::vector<float> embed(const std::string& text) const override {
        PYBIND11_OVERRIDE_PURE(std::vector<float>, zcgvs::QueryEmbedder, embed, text);
    }
    std::vector<int> lexicalTerms(const std::string& text) const override {
        PYBIND11_OVERRIDE_NAME(std::vector<int>, zcgvs::QueryEmbedder, "lexical_terms", lexicalTerms, text);
    }
};

// [rows, dim] view of a 1-D (one row) or 2-D float32 array.
std::pair<int, int> rowsOf(const FloatRows& a) {
    if (a.ndim() == 1) {
        return {1, static_cast<int>(a.shape(0))};
    }
    if (a.ndim() == 2) {
        return {static_cast<int>(a.shape(0)), static_cast<int>(a.shape(1))};
    }
    throw std::invalid_argument("zcgvs: expected a [dim] or [rows, dim] float32 array");
}

zcgvs::ScalarType dtypeOf(const std::string& name) {
    if (name == "float32") return zcgvs::ScalarType::Float32;
    if (name == "float16") return zcgvs::ScalarType::Float16;
    if (name == "int8") return zcgvs::ScalarType::Int8;
    if (name == "binary") return zcgvs::ScalarType::Binary;
    throw std::invalid_argument("zcgvs: unknown storage dtype '" + name + "'");
}

}  // namespace

PYBIND11_MODULE(zcgvs_engine, module) {
    module.doc() = "Zero-Copy GPU Vector Search & Re-Ranking Engine (MI355X build)";

    py::register_exception<zcgvs::HipError>(module, "HipError", PyExc_RuntimeError);

    py::enum_<zcgvs::Metric>(module, "Metric")
        .value("Cosine", zcgvs::Metric::Cosine)
        .value("DotProduct", zcgvs::Metric::DotProduct)
        .value("L2", zcgvs::Metric::L2);

    py::enum_<zcgvs::RerankerBackend>(module, "RerankerBackend").value("Onnx", zcgvs::RerankerBackend::Onnx);

    py::enum_<zcgvs::SimilarityBackend>(module, "SimilarityBackend")
        .value("Custom", zcgvs::SimilarityBackend::Custom)
        .value("Cublas", zcgvs::SimilarityBackend::Cublas);

    py::class_<zcgvs::EngineConfig>(module, "EngineConfig")
        .def(py::init<>())
        .def_readwrite("embeddings_path", &zcgvs::EngineConfig::embeddings_path)
        .def_readwrite("metadata_path", &zcgvs::EngineConfig::metadata_path)
        .def_readwrite("vocab_path", &zcgvs::EngineConfig::vocab_path)
        .def_readwrite("rescore_embeddings_path", &zcgvs::EngineConfig::rescore_embeddings_path)
        .def_readwrite("lexical_index_path", &zcgvs::EngineConfig::lexical_index_path)
        .def_readwrite("encoder_model_path", &zcgvs::EngineConfig::encoder_model_path)
        .def_readwrite("encoder_output_name", &zcgvs::EngineConfig::encoder_output_name)
        .def_readwrite("encoder_max_seq_len", &zcgvs::EngineConfig::encoder_max_seq_len)
        .def_readwrite("reranker_backend", &zcgvs::EngineConfig::reranker_backend)
        .def_readwrite("reranker_model_path", &zcgvs::EngineConfig::reranker_model_path)
        .def_readwrite("reranker_output_name", &zcgvs::EngineConfig::reranker_output_name)
        .def_readwrite("reranker_max_seq_len", &zcgvs::EngineConfig::reranker_max_seq_len)
        .def_readwrite("reranker_batch_size", &zcgvs::EngineConfig::reranker_batch_size)
        .def_readwrite("device_id", &zcgvs::EngineConfig::device_id)
        .def_readwrite("lowercase", &zcgvs::EngineConfig::lowercase)
        .def_readwrite("metric", &zcgvs::EngineConfig::metric)
        .def_readwrite("similarity_backend", &zcgvs::EngineConfig::similarity_backend)
        .def_readwrite("default_top_k", &zcgvs::EngineConfig::default_top_k)
        .def_readwrite("default_candidates", &zcgvs::EngineConfig::default_candidates)
        .def_readwrite("rescore_candidates", &zcgvs::EngineConfig::rescore_candidates)
        .def_readwrite("hybrid", &zcgvs::EngineConfig::hybrid)
        .def_readwrite("dense_weight", &zcgvs::EngineConfig::dense_weight)
        .def_readwrite("max_query_terms", &zcgvs::EngineConfig::max_query_terms)
        .def_readwrite("use_cuda_graphs", &zcgvs::EngineConfig::use_cuda_graphs);

    py::class_<zcgvs::SearchOptions>(module, "SearchOptions")
        .def(py::init<>())
        .def_readwrite("top_k", &zcgvs::SearchOptions::top_k)
        .def_readwrite("candidates", &zcgvs::SearchOptions::candidates)
        .def_readwrite("use_config_metric", &zcgvs::SearchOptions::use_config_metric)
        .def_readwrite("metric", &zcgvs::SearchOptions::metric)
        .def_readwrite("allow", &zcgvs::SearchOptions::allow)
        .def_readwrite("rescore_candidates", &zcgvs::SearchOptions::rescore_candidates)
        .def_readwrite("dense_weight", &zcgvs::SearchOptions::dense_weight)
        .def_readwrite("hybrid", &zcgvs::SearchOptions::hybrid)
        .def_readwrite("rerank", &zcgvs::SearchOptions::rerank)
        .def_readwrite("use_config_backend", &zcgvs::SearchOptions::use_config_backend)
        .def_readwrite("backend", &zcgvs::SearchOptions::backend)
        .def_readwrite("use_config_graphs", &zcgvs::SearchOptions::use_config_graphs)
        .def_readwrite("use_graph", &zcgvs::SearchOptions::use_graph);

    py::class_<zcgvs::SearchHit>(module, "SearchHit")
        .def_readonly("doc_id", &zcgvs::SearchHit::doc_id)
        .def_readonly("text", &zcgvs::SearchHit::text)
        .def_readonly("similarity", &zcgvs::SearchHit::similarity)
        .def_readonly("rerank_score", &zcgvs::SearchHit::rerank_score)
        .def_readonly("corpus_index", &zcgvs::SearchHit::corpus_index)
        .def("__repr__", [](const zcgvs::SearchHit& hit) {
            return "<SearchHit doc_id='" + hit.doc_id + "' rerank_score=" + std::to_string(hit.rerank_score) + ">";
        });

    py::class_<zcgvs::Candidate>(module, "Candidate")
        .def_readonly("doc_id", &zcgvs::Candidate::doc_id)
        .def_readonly("score", &zcgvs::Candidate::score)
        .def_readonly("corpus_index", &zcgvs::Candidate::corpus_index)
        .def("__repr__", [](const zcgvs::Candidate& c) {
            return "<Candidate doc_id='" + c.doc_id + "' score=" + std::to_string(c.score) + ">";
        });

    py::class_<zcgvs::SearchTiming>(module, "SearchTiming")
        .def_readonly("tokenize_ms", &zcgvs::SearchTiming::tokenize_ms)
        .def_readonly("embed_ms", &zcgvs::SearchTiming::embed_ms)
        .def_readonly("search_gpu_ms", &zcgvs::SearchTiming::search_gpu_ms)
        .def_readonly("copy_ms", &zcgvs::SearchTiming::copy_ms)
        .def_readonly("rerank_ms", &zcgvs::SearchTiming::rerank_ms)
        .def_readonly("total_ms", &zcgvs::SearchTiming::total_ms)
        .def_readonly("batch", &zcgvs::SearchTiming::batch)
        .def_readonly("graph_replay", &zcgvs::SearchTiming::graph_replay)
        .def("__repr__", [](const zcgvs::SearchTiming& t) {
            return "<SearchTiming total_ms=" + std::to_string(t.total_ms) + " gpu_ms=" + std::to_string(t.search_gpu_ms) +
                   ">";
        });

    py::class_<zcgvs::SearchResponse>(module, "SearchResponse")
        .def_readonly("hits", &zcgvs::SearchResponse::hits)
        .def_readonly("timing", &zcgvs::SearchResponse::timing);

    py::class_<zcgvs::BatchSearchResponse>(module, "BatchSearchResponse")
        .def_readonly("results", &zcgvs::BatchSearchResponse::results)
        .def_readonly("timing", &zcgvs::BatchSearchResponse::timing);

    py::class_<zcgvs::EngineStats>(module, "EngineStats")
        .def_readonly("corpus_size", &zcgvs::EngineStats::corpus_size)
        .def_readonly("dim", &zcgvs::EngineStats::dim)
        .def_readonly("storage_dtype", &zcgvs::EngineStats::storage_dtype)
        .def_readonly("corpus_bytes", &zcgvs::EngineStats::corpus_bytes)
        .def_readonly("has_rescore_store", &zcgvs::EngineStats::has_rescore_store)
        .def_readonly("rescore_dtype", &zcgvs::EngineStats::rescore_dtype)
        .def_readonly("rescore_bytes", &zcgvs::EngineStats::rescore_bytes)
        .def_readonly("has_lexical_index", &zcgvs::EngineStats::has_lexical_index)
        .def_readonly("lexical_postings", &zcgvs::EngineStats::lexical_postings)
        .def_readonly("lexical_bytes", &zcgvs::EngineStats::lexical_bytes)
        .def_readonly("has_reranker", &zcgvs::EngineStats::has_reranker)
        .def_readonly("graph_captures", &zcgvs::EngineStats::graph_captures)
        .def_readonly("graph_launches", &zcgvs::EngineStats::graph_launches)
        .def_readonly("device_name", &zcgvs::EngineStats::device_name)
        .def_readonly("device_total_memory", &zcgvs::EngineStats::device_total_memory)
        .def_readonly("compute_major", &zcgvs::EngineStats::compute_major)
        .def_readonly("compute_minor", &zcgvs::EngineStats::compute_minor);

    py::class_<zcgvs::QueryEmbedder, PyQueryEmbedder, std::shared_ptr<zcgvs::QueryEmbedder>>(module, "QueryEmbedder")
        .def(py::init<>())
        .def("embed", &zcgvs::QueryEmbedder::embed)
        .def("lexical_terms", &zcgvs::QueryEmbedder::lexicalTerms);

    // Artifacts (device-resident). Writers produce the reference's on-disk layouts.
    py::class_<zcgvs::EmbeddingStore, std::unique_ptr<zcgvs::EmbeddingStore>>(module, "EmbeddingStore")
        .def_static("load", &zcgvs::EmbeddingStore::loadFromFile, py::arg("path"),
                    py::call_guard<py::gil_scoped_release>())
        .def_static(
            "from_numpy",
            [](const FloatRows& rows, const std::string& dtype, float scale, bool normalized, bool per_row) {
                const auto shape = rowsOf(rows);
                if (per_row) {
                    return zcgvs::EmbeddingStore::fromHostMatrixPerRow(rows.data(), shape.first, shape.second, normalized);
                }
                return zcgvs::EmbeddingStore::fromHostMatrix(rows.data(), shape.first, shape.second, dtypeOf(dtype), scale,
                                                             normalized);
            },
            py::arg("rows"), py::arg("dtype") = "float32", py::arg("scale") = 1.0f, py::arg("normalized") = true,
            py::arg("per_row_scales") = false)
        .def("save", &zcgvs::EmbeddingStore::saveToFile, py::arg("path"), py::call_guard<py::gil_scoped_release>())
        .def_property_readonly("doc_count", &zcgvs::EmbeddingStore::docCount)
        .def_property_readonly("dim", &zcgvs::EmbeddingStore::dim)
        .def_property_readonly("dtype", [](const zcgvs::EmbeddingStore& s) { return std::string(zcgvs::scalarName(s.dtype())); })
        .def_property_readonly("scale", &zcgvs::EmbeddingStore::scale)
        .def_property_readonly("normalized", &zcgvs::EmbeddingStore::normalized)
        .def_property_readonly("has_row_scales", &zcgvs::EmbeddingStore::hasRowScales)
        .def_property_readonly("device_bytes", &zcgvs::EmbeddingStore::deviceBytes);

    py::class_<zcgvs::LexicalIndex, std::unique_ptr<zcgvs::LexicalIndex>>(module, "LexicalIndex")
        .def_static("load", &zcgvs::LexicalIndex::loadFromFile, py::arg("path"), py::call_guard<py::gil_scoped_release>())
        .def_static(
            "from_csr",
            [](py::array_t<std::int64_t, py::array::c_style | py::array::forcecast> offsets,
               py::array_t<int, py::array::c_style | py::array::forcecast> docs, FloatRows weights, std::int64_t doc_count,
               float k1, float b, float avgdl) {
                const int vocab = static_cast<int>(offsets.size()) - 1;
                if (vocab <= 0 || docs.size() != weights.size()) {
                    throw std::invalid_argument("zcgvs: from_csr needs vocab + 1 offsets and equal-length postings");
                }
                return zcgvs::LexicalIndex::fromHostCsr(offsets.data(), docs.data(), weights.data(), doc_count, vocab, k1, b,
                                                        avgdl);
            },
            py::arg("offsets"), py::arg("docs"), py::arg("weights"), py::arg("doc_count"), py::arg("k1") = 1.2f,
            py::arg("b") = 0.75f, py::arg("avg_doc_len") = 0.0f)
        .def("save", &zcgvs::LexicalIndex::saveToFile, py::arg("path"), py::call_guard<py::gil_scoped_release>())
        .def_property_readonly("doc_count", &zcgvs::LexicalIndex::docCount)
        .def_property_readonly("posting_count", &zcgvs::LexicalIndex::postingCount)
        .def_property_readonly("vocab_size", &zcgvs::LexicalIndex::vocabSize)
        .def_property_readonly("k1", &zcgvs::LexicalIndex::k1)
        .def_property_readonly("b", &zcgvs::LexicalIndex::b)
        .def_property_readonly("avg_doc_len", &zcgvs::LexicalIndex::averageDocLength)
        .def_property_readonly("postings_sorted", &zcgvs::LexicalIndex::postingsSorted)
        .def_property_readonly("has_slice_table",
                               [](const zcgvs::LexicalIndex& index) { return index.deviceSliceTable() != nullptr; })
        .def_property_readonly("device_bytes", &zcgvs::LexicalIndex::deviceBytes);

    module.def("write_metadata", &zcgvs::Corpus::saveMetadata, py::arg("path"), py::arg("ids"), py::arg("texts"));

    py::class_<zcgvs::Engine>(module, "Engine")
        .def(py::init<const zcgvs::EngineConfig&>(), py::arg("config"), py::call_guard<py::gil_scoped_release>())
        .def(
            "set_query_embedder",
            [](zcgvs::Engine& engine, std::shared_ptr<zcgvs::QueryEmbedder> embedder) {
                engine.setQueryEmbedder(std::move(embedder));
            },
            py::arg("embedder"), py::keep_alive<1, 2>())
        .def(
            "search_vectors",
            [](const zcgvs::Engine& engine, const FloatRows& queries, const zcgvs::SearchOptions* options,
               const std::vector<std::vector<int>>& terms) {
                const auto shape = rowsOf(queries);
                const zcgvs::SearchOptions opts = options != nullptr ? *options : engine.defaultOptions();
                py::gil_scoped_release release;
                return engine.searchVectors(queries.data(), shape.first, shape.second, opts, terms);
            },
            py::arg("queries"), py::arg("options") = nullptr, py::arg("terms") = std::vector<std::vector<int>>{})
        .def(
            "retrieve_vectors",
            [](const zcgvs::Engine& engine, const FloatRows& query, int k, zcgvs::Metric metric,
               const std::vector<int>& allow) {
                const auto shape = rowsOf(query);
                if (shape.first != 1) {
                    throw std::invalid_argument("zcgvs: retrieve_vectors takes one query");
                }
                py::gil_scoped_release release;
                return engine.retrieveVectors(query.data(), shape.second, k, metric, allow);
            },
            py::arg("query"), py::arg("k"), py::arg("metric") = zcgvs::Metric::Cosine,
            py::arg("allow") = std::vector<int>{})
        .def(
            "add_vectors",
            [](zcgvs::Engine& engine, const std::vector<std::string>& ids, const std::vector<std::string>& texts,
               const FloatRows& vectors) {
                const auto shape = rowsOf(vectors);
                if (shape.second != engine.dim()) {
                    throw std::invalid_argument("zcgvs: vector dim does not match the corpus");
                }
                py::gil_scoped_release release;
                engine.addVectors(ids, texts, vectors.data(), shape.first);
            },
            py::arg("ids"), py::arg("texts"), py::arg("vectors"))
        .def(
            "search",
            [](const zcgvs::Engine& engine, const std::string& query, int top_k, int candidates) {
                return engine.search(query, top_k, candidates);
            },
            py::arg("query"), py::arg("top_k"), py::arg("candidates"), py::call_guard<py::gil_scoped_release>())
        .def(
            "search", [](const zcgvs::Engine& engine, const std::string& query) { return engine.search(query); },
            py::arg("query"), py::call_guard<py::gil_scoped_release>())
        .def(
            "search_timed",
            [](const zcgvs::Engine& engine, const std::string& query, int top_k, int candidates, zcgvs::Metric metric,
               const std::vector<int>& allow) { return engine.searchTimed(query, top_k, candidates, metric, allow); },
            py::arg("query"), py::arg("top_k"), py::arg("candidates"), py::arg("metric") = zcgvs::Metric::Cosine,
            py::arg("allow") = std::vector<int>{}, py::call_guard<py::gil_scoped_release>())
        .def(
            "search_with",
            [](const zcgvs::Engine& engine, const std::string& query, const zcgvs::SearchOptions& options) {
                return engine.searchTimed(query, options);
            },
            py::arg("query"), py::arg("options"), py::call_guard<py::gil_scoped_release>())
        .def(
            "search_batch",
            [](const zcgvs::Engine& engine, const std::vector<std::string>& queries, const zcgvs::SearchOptions& options) {
                return engine.searchBatch(queries, options);
            },
            py::arg("queries"), py::arg("options"), py::call_guard<py::gil_scoped_release>())
        .def(
            "retrieve",
            [](const zcgvs::Engine& engine, const std::string& query, int k, zcgvs::Metric metric,
               const std::vector<int>& allow) { return engine.retrieve(query, k, metric, allow); },
            py::arg("query"), py::arg("k"), py::arg("metric") = zcgvs::Metric::Cosine,
            py::arg("allow") = std::vector<int>{}, py::call_guard<py::gil_scoped_release>())
        .def(
            "add_documents",
            [](zcgvs::Engine& engine, const std::vector<std::string>& ids, const std::vector<std::string>& texts) {
                engine.addDocuments(ids, texts);
            },
            py::arg("ids"), py::arg("texts"), py::call_guard<py::gil_scoped_release>())
        .def("default_options", &zcgvs::Engine::defaultOptions)
        .def("stats", &zcgvs::Engine::stats, py::call_guard<py::gil_scoped_release>())
        .def_property_readonly("corpus_size", &zcgvs::Engine::corpusSize)
        .def_property_readonly("dim", &zcgvs::Engine::dim)
        .def_property_readonly("storage_dtype", &zcgvs::Engine::storageDtype)
        .def_property_readonly("has_lexical_index", &zcgvs::Engine::hasLexicalIndex)
        .def_property_readonly("has_rescore_store", &zcgvs::Engine::hasRescoreStore)
        .def_property_readonly("has_reranker", &zcgvs::Engine::hasReranker)
        .def_property_readonly("has_query_embedder", &zcgvs::Engine::hasQueryEmbedder);
}
