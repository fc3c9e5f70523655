// Searcher over the fused C-ABI pipeline (src/search/searcher.cpp).
#include "zcgvs/search/searcher.hpp"

#include "zcgvs/core/trace_range.hpp"

#include <algorithm>
#include <cstring>
#include <stdexcept>
#include <string>

namespace zcgvs {

namespace {

template <typename Buffer>
bool grow(Buffer& buffer, std::size_t required) {
    if (buffer.size() >= required) {
        return false;
    }
    buffer.allocate(required);
    return true;
}

zcgvs_store_desc storeDesc(const EmbeddingStore& store) {
    zcgvs_store_desc desc{};
    desc.data = store.deviceData();
    desc.doc_count = store.docCount();
    desc.dim = store.dim();
    desc.dtype = static_cast<int>(store.dtype());
    desc.scale = store.scale();
    desc.row_scales = store.deviceRowScales();
    return desc;
}

// Rethrows a failed status with the message captured before any later call could replace it.
[[noreturn]] void raise(int status, const std::string& message) {
    if (status == ZCGVS_ERR_INVALID_ARGUMENT) {
        throw std::invalid_argument(message);
    }
    throw HipError(message);
}

std::size_t workspaceBytes(const zcgvs_search_desc& desc) {
    const std::size_t bytes = zcgvs_search_workspace_bytes(&desc);
    if (bytes == 0) {
        const std::string message = zcgvs_last_error();
        if (message.find("exceeds the supported document count") != std::string::npos) {
            throw std::runtime_error(message);
        }
        throw std::invalid_argument(message.empty() ? "zcgvs: invalid search descriptor" : message);
    }
    return bytes;
}

}  // namespace

bool Searcher::GraphKey::operator==(const GraphKey& other) const {
    return corpus == other.corpus && row_scales == other.row_scales &&
           rescore_corpus == other.rescore_corpus && lexical_index == other.lexical_index &&
           queries == other.queries && mask == other.mask && generation == other.generation &&
           doc_count == other.doc_count && k == other.k && batch == other.batch &&
           rescore_candidates == other.rescore_candidates && lexical_stride == other.lexical_stride &&
           metric == other.metric && dense_weight == other.dense_weight;
}

Searcher::Searcher(const EmbeddingStore& store) : store_(store), dim_(store.dim()) {}

Searcher::~Searcher() { destroyGraph(); }

void Searcher::destroyGraph() noexcept {
    if (graph_ != nullptr) {
        zcgvs_graph_destroy(graph_);
        graph_ = nullptr;
    }
}

void Searcher::setRescoreStore(const EmbeddingStore* store) {
    if (store != nullptr) {
        if (store->dim() != dim_) {
            throw std::invalid_argument("zcgvs: rescore store dim does not match the corpus");
        }
        if (store->dtype() == ScalarType::Binary) {
            throw std::invalid_argument("zcgvs: rescore store must not be binary");
        }
    }
    rescore_store_ = store;
    destroyGraph();
}

void Searcher::setLexicalIndex(const LexicalIndex* index) {
    lexical_index_ = index;
    destroyGraph();
}

bool Searcher::rescoreEnabled(const SearchParams& params) const {
    return rescore_store_ != nullptr && params.rescore_candidates > 0;
}

bool Searcher::lexicalEnabled(const SearchParams& params) const {
    return lexical_index_ != nullptr && params.lexical_stride > 0 && params.host_query_terms != nullptr;
}

// The argument checks of src/search/searcher.cpp:91-135, with the same messages and types.
void Searcher::validate(int dim, int batch, const SearchParams& params, std::int64_t doc_count) const {
    if (dim != dim_) {
        throw std::invalid_argument("zcgvs: query dim " + std::to_string(dim) + " does not match corpus dim " +
                                    std::to_string(dim_));
    }
    if (batch <= 0) {
        throw std::invalid_argument("zcgvs: batch must be positive");
    }
    if (params.k <= 0) {
        throw std::invalid_argument("zcgvs: k must be positive");
    }
    if (doc_count > static_cast<std::int64_t>(INT32_MAX)) {
        throw std::runtime_error("zcgvs: corpus exceeds the supported document count");
    }
    const int max_k = zcgvs_topk_max_k();
    if (params.k > doc_count) {
        throw std::invalid_argument("zcgvs: k=" + std::to_string(params.k) + " exceeds corpus size " +
                                    std::to_string(doc_count));
    }
    if (params.k > max_k) {
        throw std::invalid_argument("zcgvs: k=" + std::to_string(params.k) + " exceeds kernel capacity " +
                                    std::to_string(max_k));
    }
    if (rescoreEnabled(params)) {
        if (params.rescore_candidates < params.k) {
            throw std::invalid_argument("zcgvs: rescore_candidates must be at least k");
        }
        if (params.rescore_candidates > doc_count) {
            throw std::invalid_argument("zcgvs: rescore_candidates exceeds corpus size");
        }
        if (params.rescore_candidates > max_k) {
            throw std::invalid_argument("zcgvs: rescore_candidates=" + std::to_string(params.rescore_candidates) +
                                        " exceeds kernel capacity " + std::to_string(max_k));
        }
        if (rescore_store_->docCount() < doc_count) {
            throw std::invalid_argument("zcgvs: rescore store holds fewer documents than the corpus");
        }
    }
    if (lexicalEnabled(params) && lexical_index_->docCount() < doc_count) {
        throw std::invalid_argument("zcgvs: lexical index holds fewer documents than the corpus");
    }
}

zcgvs_search_desc Searcher::describe(const float* queries, int batch, const SearchParams& params) const {
    zcgvs_search_desc desc{};
    desc.corpus = storeDesc(store_);
    desc.queries = queries;
    desc.batch = batch;
    desc.k = params.k;
    desc.metric = static_cast<int>(params.metric);
    desc.int8_mode = store_.hasRowScales() ? ZCGVS_INT8_PER_VECTOR : ZCGVS_INT8_REFERENCE;
    desc.mask = params.d_mask;
    desc.dense_weight = 1.0f;
    if (rescoreEnabled(params)) {
        desc.rescore = storeDesc(*rescore_store_);
        desc.rescore_candidates = params.rescore_candidates;
    }
    if (lexicalEnabled(params)) {
        desc.lex_offsets = lexical_index_->deviceOffsets();
        desc.lex_docs = lexical_index_->devicePostingDocs();
        desc.lex_weights = lexical_index_->devicePostingWeights();
        desc.lex_doc_count = lexical_index_->docCount();
        desc.lex_vocab_size = lexical_index_->vocabSize();
        if (lexical_index_->postingsSorted()) {  // checked when the index was loaded
            desc.flags |= ZCGVS_SEARCH_SORTED_POSTINGS;
            desc.lex_slice_table = lexical_index_->deviceSliceTable();
        }
        desc.query_terms = d_query_terms_.data();
        desc.lexical_stride = params.lexical_stride;
        desc.dense_weight = params.dense_weight;
    }
    return desc;
}

void Searcher::ensureCapacity(int batch, const SearchParams& params, const zcgvs_search_desc& desc) {
    const std::size_t results = static_cast<std::size_t>(batch) * static_cast<std::size_t>(params.k);
    bool moved = false;
    moved |= grow(d_out_indices_, results);
    moved |= grow(d_out_values_, results);
    moved |= grow(d_workspace_, workspaceBytes(desc));
    if (moved) {
        ++generation_;
        destroyGraph();
    }
}

void Searcher::search(const float* host_queries, int dim, int batch, const SearchParams& params,
                      const HipStream& stream) {
    validate(dim, batch, params, store_.docCount());
    if (host_queries == nullptr) {
        throw std::invalid_argument("zcgvs: queries must not be null");
    }
    const std::size_t elements = static_cast<std::size_t>(batch) * static_cast<std::size_t>(dim_);
    if (grow(d_queries_, elements)) {
        ++generation_;
        destroyGraph();
    }
    if (h_queries_.size() < elements) {
        h_queries_.allocate(elements);
    }
    std::memcpy(h_queries_.data(), host_queries, elements * sizeof(float));
    d_queries_.copyFromHost(h_queries_.data(), elements, stream.get());
    run(d_queries_.data(), dim, batch, params, stream);
}

void Searcher::searchDevice(const float* device_queries, int dim, int batch, const SearchParams& params,
                            const HipStream& stream) {
    if (device_queries == nullptr) {
        throw std::invalid_argument("zcgvs: queries must not be null");
    }
    run(device_queries, dim, batch, params, stream);
}

void Searcher::run(const float* device_queries, int dim, int batch, const SearchParams& params,
                   const HipStream& stream) {
    ZCGVS_TRACE_RANGE("zcgvs::search");
    validate(dim, batch, params, store_.docCount());
    if (lexicalEnabled(params)) {
        const std::size_t terms = static_cast<std::size_t>(batch) * static_cast<std::size_t>(params.lexical_stride);
        if (grow(d_query_terms_, terms)) {
            ++generation_;
            destroyGraph();
        }
        if (h_query_terms_.size() < terms) {
            h_query_terms_.allocate(terms);
        }
        std::memcpy(h_query_terms_.data(), params.host_query_terms, terms * sizeof(int));
        d_query_terms_.copyFromHost(h_query_terms_.data(), terms, stream.get());
    }
    const zcgvs_search_desc desc = describe(device_queries, batch, params);
    ensureCapacity(batch, params, desc);
    const std::size_t workspace = d_workspace_.size();

    const bool use_graph = params.use_graph;
    if (use_graph) {
        GraphKey key;
        key.corpus = desc.corpus.data;
        key.row_scales = desc.corpus.row_scales;
        key.rescore_corpus = desc.rescore.data;
        key.lexical_index = desc.lex_offsets;
        key.queries = device_queries;
        key.mask = params.d_mask;
        key.generation = generation_;
        key.doc_count = desc.corpus.doc_count;
        key.k = params.k;
        key.batch = batch;
        key.rescore_candidates = desc.rescore_candidates;
        key.lexical_stride = desc.lexical_stride;
        key.metric = desc.metric;
        key.dense_weight = desc.dense_weight;
        if (graph_ == nullptr || !(key == graph_key_)) {
            destroyGraph();
            // drain this request's uploads so the graph holds the pipeline and nothing else
            stream.synchronize();
            check(zcgvs_graph_begin_capture(stream.get()));
            const int status = zcgvs_search_topk(&desc, d_workspace_.data(), workspace, d_out_indices_.data(),
                                                 d_out_values_.data(), stream.get());
            const std::string message = status == ZCGVS_OK ? std::string() : zcgvs_last_error();
            zcgvs_graph_t graph = nullptr;
            const int ended = zcgvs_graph_end_capture(stream.get(), &graph);
            if (status != ZCGVS_OK) {
                if (graph != nullptr) {
                    zcgvs_graph_destroy(graph);
                }
                raise(status, message);
            }
            check(ended);
            graph_ = graph;
            graph_key_ = key;
            ++graph_captures_;
        }
    }

    ev_start_.record(stream.get());
    if (use_graph) {
        check(zcgvs_graph_launch(graph_, stream.get()));
        ++graph_launches_;
    } else {
        check(zcgvs_search_topk(&desc, d_workspace_.data(), workspace, d_out_indices_.data(), d_out_values_.data(),
                                stream.get()));
    }
    ev_end_.record(stream.get());

    last_desc_ = desc;
    used_graph_ = use_graph;
    current_k_ = params.k;
    current_batch_ = batch;
}

HostTopK Searcher::copyResultToHost(const HipStream& stream) {
    ZCGVS_TRACE_RANGE("zcgvs::copyResultToHost");
    if (current_k_ == 0 || current_batch_ == 0) {
        throw std::runtime_error("zcgvs: copyResultToHost called before search");
    }
    const std::size_t elements = static_cast<std::size_t>(current_batch_) * static_cast<std::size_t>(current_k_);
    if (h_out_indices_.size() < elements) {
        h_out_indices_.allocate(elements);
        h_out_values_.allocate(elements);
    }
    if (h_overflow_.size() < static_cast<std::size_t>(current_batch_)) {
        h_overflow_.allocate(static_cast<std::size_t>(current_batch_));
    }
    d_out_indices_.copyToHost(h_out_indices_.data(), elements, stream.get());
    d_out_values_.copyToHost(h_out_values_.data(), elements, stream.get());
    std::uint32_t* flags = nullptr;
    check(zcgvs_search_overflow_flags(&last_desc_, d_workspace_.data(), &flags));
    check(zcgvs_memcpy_d2h(h_overflow_.data(), flags, static_cast<std::size_t>(current_batch_) * sizeof(std::uint32_t),
                           stream.get()));
    stream.synchronize();
    last_gpu_ms_ = static_cast<double>(ev_end_.elapsedSince(ev_start_));

    // the device already replaced these queries' results with its exact fallback's
    for (int q = 0; q < current_batch_; ++q) {
        exact_recomputes_ += h_overflow_.data()[q] != 0u ? 1u : 0u;
    }

    HostTopK result;
    result.batch = current_batch_;
    result.k = current_k_;
    result.indices.assign(h_out_indices_.data(), h_out_indices_.data() + elements);
    result.scores.assign(h_out_values_.data(), h_out_values_.data() + elements);
    return result;
}

}  // namespace zcgvs
