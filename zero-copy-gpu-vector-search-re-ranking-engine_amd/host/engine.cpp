// Engine: option resolution, masks, result assembly and the request paths of
// src/engine/engine.cpp, over the Searcher.
#include "zcgvs/engine/engine.hpp"

#include "zcgvs/core/trace_range.hpp"

#include <algorithm>
#include <chrono>
#include <stdexcept>
#include <unordered_set>

namespace zcgvs {

namespace {

using Clock = std::chrono::steady_clock;

double msSince(Clock::time_point begin) {
    return std::chrono::duration<double, std::milli>(Clock::now() - begin).count();
}

}  // namespace

Engine::Engine(const EngineConfig& config) : config_(config) {
    setDevice(config_.device_id);
    corpus_ = Corpus::load(config_.embeddings_path, config_.metadata_path);
    if (!config_.rescore_embeddings_path.empty()) {
        rescore_store_ = std::make_unique<EmbeddingStore>(EmbeddingStore::loadFromFile(config_.rescore_embeddings_path));
    }
    if (!config_.lexical_index_path.empty()) {
        lexical_index_ = std::make_unique<LexicalIndex>(LexicalIndex::loadFromFile(config_.lexical_index_path));
    }
    attach();
}

Engine::Engine(const EngineConfig& config, Corpus corpus, std::unique_ptr<EmbeddingStore> rescore,
               std::unique_ptr<LexicalIndex> lexical)
    : config_(config), corpus_(std::move(corpus)), rescore_store_(std::move(rescore)),
      lexical_index_(std::move(lexical)) {
    setDevice(config_.device_id);
    attach();
}

Engine::~Engine() = default;

void Engine::attach() {
    stream_ = std::make_unique<HipStream>();
    searcher_ = std::make_unique<Searcher>(corpus_.embeddings());
    if (rescore_store_ != nullptr) {
        if (rescore_store_->docCount() < corpus_.size()) {
            throw std::runtime_error("zcgvs: the rescore store holds fewer documents than the primary corpus");
        }
        searcher_->setRescoreStore(rescore_store_.get());
    }
    if (lexical_index_ != nullptr) {
        if (lexical_index_->docCount() < corpus_.size()) {
            throw std::runtime_error("zcgvs: the lexical index holds fewer documents than the corpus");
        }
        searcher_->setLexicalIndex(lexical_index_.get());
    }
}

void Engine::setQueryEmbedder(std::shared_ptr<const QueryEmbedder> embedder) {
    std::lock_guard<std::mutex> lock(mutex_);
    embedder_ = std::move(embedder);
}

const QueryEmbedder& Engine::embedder() const {
    if (embedder_ == nullptr) {
        throw std::runtime_error(
            "zcgvs: text queries need a query embedder (setQueryEmbedder / set_query_embedder); "
            "ONNX encoding is not part of this build, use search_vectors with embedded queries");
    }
    return *embedder_;
}

std::int64_t Engine::corpusSize() const { return corpus_.size(); }

std::string Engine::storageDtype() const { return scalarName(corpus_.embeddings().dtype()); }

SearchOptions Engine::defaultOptions() const {
    SearchOptions options;
    options.top_k = config_.default_top_k;
    options.candidates = config_.default_candidates;
    options.use_config_metric = true;
    options.rescore_candidates = -1;
    options.dense_weight = -1.0f;
    options.hybrid = config_.hybrid && lexical_index_ != nullptr;
    options.rerank = false;  // no cross-encoder in this build
    options.use_config_backend = true;
    options.use_config_graphs = true;
    return options;
}

// Option resolution of src/engine/engine.cpp:87-128.
Engine::Resolved Engine::resolve(const SearchOptions& options, std::int64_t corpus_size) const {
    Resolved r;
    r.top_k = options.top_k > 0 ? options.top_k : config_.default_top_k;
    r.candidates = options.candidates > 0 ? options.candidates : config_.default_candidates;
    r.metric = options.use_config_metric ? config_.metric : options.metric;
    r.use_graph = options.use_config_graphs ? config_.use_cuda_graphs : options.use_graph;
    r.hybrid = options.hybrid && lexical_index_ != nullptr;
    r.dense_weight = options.dense_weight >= 0.0f ? options.dense_weight : config_.dense_weight;
    r.dense_weight = std::min(1.0f, std::max(0.0f, r.dense_weight));
    if (r.top_k <= 0) {
        throw std::invalid_argument("zcgvs: top_k must be positive");
    }
    r.candidates = std::max(r.top_k, r.candidates);
    if (r.candidates > corpus_size) {
        r.candidates = static_cast<int>(corpus_size);
    }
    if (r.top_k > r.candidates) {
        r.top_k = r.candidates;
    }
    if (rescore_store_ != nullptr) {
        const int requested = options.rescore_candidates >= 0 ? options.rescore_candidates : config_.rescore_candidates;
        r.rescore_candidates = std::max(requested, 0);
        if (r.rescore_candidates > 0) {
            r.rescore_candidates = std::max(r.rescore_candidates, r.candidates);
            if (r.rescore_candidates > corpus_size) {
                r.rescore_candidates = static_cast<int>(corpus_size);
            }
        }
    }
    return r;
}

const std::uint8_t* Engine::buildMask(const std::vector<int>& allow_ids, std::int64_t doc_count) const {
    if (allow_ids.empty()) {
        return nullptr;
    }
    host_mask_.assign(static_cast<std::size_t>(doc_count), 0);
    for (const int index : allow_ids) {
        if (index >= 0 && index < doc_count) {
            host_mask_[static_cast<std::size_t>(index)] = 1;
        }
    }
    if (d_mask_.size() < static_cast<std::size_t>(doc_count)) {
        d_mask_.allocate(static_cast<std::size_t>(doc_count));
    }
    d_mask_.copyFromHost(host_mask_.data(), static_cast<std::size_t>(doc_count), stream_->get());
    return d_mask_.data();
}

// Query term ids without repeats or negatives, capped at max_query_terms (src/engine/
// engine.cpp:150-173 applied to ids).
std::vector<int> Engine::dedupeTerms(const std::vector<int>& terms) const {
    std::vector<int> out;
    std::unordered_set<int> seen;
    const int limit = std::max(1, config_.max_query_terms);
    for (const int id : terms) {
        if (id < 0 || !seen.insert(id).second) {
            continue;
        }
        out.push_back(id);
        if (static_cast<int>(out.size()) >= limit) {
            break;
        }
    }
    return out;
}

// Hits of one query in selection order. With no cross-encoder the rerank score is the
// similarity, and a stable sort keeps the (score desc, index asc) order of the selection.
std::vector<SearchHit> Engine::assemble(const HostTopK& selection, int query, const Resolved& resolved) const {
    const std::int64_t n = corpus_.size();
    const std::size_t base = selection.offset(query);
    std::vector<SearchHit> hits;
    hits.reserve(static_cast<std::size_t>(selection.k));
    for (int i = 0; i < selection.k; ++i) {
        const int index = selection.indices[base + static_cast<std::size_t>(i)];
        if (index < 0 || index >= n) {
            continue;
        }
        SearchHit hit;
        hit.corpus_index = index;
        hit.doc_id = corpus_.docId(index);
        hit.text = corpus_.text(index);
        hit.similarity = selection.scores[base + static_cast<std::size_t>(i)];
        hit.rerank_score = hit.similarity;
        hits.push_back(std::move(hit));
    }
    std::stable_sort(hits.begin(), hits.end(),
                     [](const SearchHit& a, const SearchHit& b) { return a.rerank_score > b.rerank_score; });
    if (static_cast<int>(hits.size()) > resolved.top_k) {
        hits.resize(static_cast<std::size_t>(resolved.top_k));
    }
    return hits;
}

BatchSearchResponse Engine::runBatch(const float* queries, int batch, const SearchOptions& options,
                                     const std::vector<std::vector<int>>& terms, double embed_ms,
                                     double tokenize_ms) const {
    ZCGVS_TRACE_RANGE("zcgvs::searchBatch");
    const auto t_start = Clock::now();
    const std::int64_t n = corpus_.size();
    const Resolved resolved = resolve(options, n);

    int stride = 0;
    std::vector<std::vector<int>> per_query;
    if (resolved.hybrid && !terms.empty()) {
        if (static_cast<int>(terms.size()) != batch) {
            throw std::invalid_argument("zcgvs: one term list per query is required");
        }
        for (const auto& t : terms) {
            per_query.push_back(dedupeTerms(t));
            stride = std::max(stride, static_cast<int>(per_query.back().size()));
        }
        if (stride > 0) {
            host_terms_.assign(static_cast<std::size_t>(batch) * static_cast<std::size_t>(stride), -1);
            for (std::size_t q = 0; q < per_query.size(); ++q) {
                std::copy(per_query[q].begin(), per_query[q].end(),
                          host_terms_.begin() + static_cast<std::ptrdiff_t>(q * static_cast<std::size_t>(stride)));
            }
        }
    }

    SearchParams params;
    params.k = resolved.candidates;
    params.metric = resolved.metric;
    params.d_mask = buildMask(options.allow, n);
    params.rescore_candidates = resolved.rescore_candidates;
    params.use_graph = resolved.use_graph;
    if (resolved.hybrid && stride > 0) {
        params.host_query_terms = host_terms_.data();
        params.lexical_stride = stride;
        params.dense_weight = resolved.dense_weight;
    }
    searcher_->search(queries, corpus_.dim(), batch, params, *stream_);
    const auto t_copy = Clock::now();
    const HostTopK selection = searcher_->copyResultToHost(*stream_);
    const double copy_ms = msSince(t_copy);

    BatchSearchResponse response;
    response.results.reserve(static_cast<std::size_t>(batch));
    for (int q = 0; q < batch; ++q) {
        response.results.push_back(assemble(selection, q, resolved));
    }
    response.timing.tokenize_ms = tokenize_ms;
    response.timing.embed_ms = embed_ms;
    response.timing.search_gpu_ms = searcher_->lastSearchGpuMs();
    response.timing.copy_ms = copy_ms;
    response.timing.rerank_ms = 0.0;
    response.timing.total_ms = msSince(t_start) + embed_ms + tokenize_ms;
    response.timing.batch = batch;
    response.timing.graph_replay = searcher_->lastSearchUsedGraph();
    return response;
}

BatchSearchResponse Engine::searchVectors(const float* queries, int batch, int dim, const SearchOptions& options,
                                          const std::vector<std::vector<int>>& terms) const {
    std::lock_guard<std::mutex> lock(mutex_);
    if (batch <= 0) {
        throw std::invalid_argument("zcgvs: searchBatch requires at least one query");
    }
    if (dim != corpus_.dim()) {
        throw std::invalid_argument("zcgvs: query dim " + std::to_string(dim) + " does not match corpus dim " +
                                    std::to_string(corpus_.dim()));
    }
    return runBatch(queries, batch, options, terms, 0.0, 0.0);
}

std::vector<Candidate> Engine::retrieveVectors(const float* query, int dim, int k, Metric metric,
                                               const std::vector<int>& allow_ids) const {
    ZCGVS_TRACE_RANGE("zcgvs::retrieve");
    std::lock_guard<std::mutex> lock(mutex_);
    if (k <= 0) {
        throw std::invalid_argument("zcgvs: k must be positive");
    }
    if (dim != corpus_.dim()) {
        throw std::invalid_argument("zcgvs: query dim " + std::to_string(dim) + " does not match corpus dim " +
                                    std::to_string(corpus_.dim()));
    }
    SearchOptions options = defaultOptions();
    options.top_k = k;
    options.candidates = k;
    options.use_config_metric = false;
    options.metric = metric;
    options.allow = allow_ids;
    options.hybrid = false;
    const Resolved resolved = resolve(options, corpus_.size());
    SearchParams params;
    params.k = resolved.candidates;
    params.metric = resolved.metric;
    params.d_mask = buildMask(allow_ids, corpus_.size());
    params.rescore_candidates = resolved.rescore_candidates;
    params.use_graph = resolved.use_graph;
    searcher_->search(query, dim, 1, params, *stream_);
    const HostTopK selection = searcher_->copyResultToHost(*stream_);
    std::vector<Candidate> out;
    for (int i = 0; i < selection.k; ++i) {
        const int index = selection.indices[static_cast<std::size_t>(i)];
        if (index < 0 || index >= corpus_.size()) {
            continue;
        }
        Candidate c;
        c.corpus_index = index;
        c.doc_id = corpus_.docId(index);
        c.score = selection.scores[static_cast<std::size_t>(i)];
        out.push_back(std::move(c));
    }
    return out;
}

BatchSearchResponse Engine::searchBatch(const std::vector<std::string>& queries, const SearchOptions& options) const {
    std::lock_guard<std::mutex> lock(mutex_);
    if (queries.empty()) {
        throw std::invalid_argument("zcgvs: searchBatch requires at least one query");
    }
    const QueryEmbedder& encoder = embedder();
    const int dim = corpus_.dim();
    const auto t_embed = Clock::now();
    std::vector<float> vectors;
    vectors.reserve(queries.size() * static_cast<std::size_t>(dim));
    for (const std::string& q : queries) {
        const std::vector<float> v = encoder.embed(q);
        if (static_cast<int>(v.size()) != dim) {
            throw std::runtime_error("zcgvs: query embedding dim does not match the corpus");
        }
        vectors.insert(vectors.end(), v.begin(), v.end());
    }
    const double embed_ms = msSince(t_embed);
    std::vector<std::vector<int>> terms;
    double tokenize_ms = 0.0;
    if (options.hybrid && lexical_index_ != nullptr) {
        const auto t_tok = Clock::now();
        for (const std::string& q : queries) {
            terms.push_back(encoder.lexicalTerms(q));
        }
        tokenize_ms = msSince(t_tok);
    }
    return runBatch(vectors.data(), static_cast<int>(queries.size()), options, terms, embed_ms, tokenize_ms);
}

SearchResponse Engine::searchTimed(const std::string& query, const SearchOptions& options) const {
    BatchSearchResponse batch = searchBatch({query}, options);
    SearchResponse response;
    response.hits = std::move(batch.results.front());
    response.timing = batch.timing;
    return response;
}

SearchResponse Engine::searchTimed(const std::string& query, int top_k, int candidates, Metric metric,
                                   const std::vector<int>& allow_ids) const {
    SearchOptions options = defaultOptions();
    options.top_k = top_k;
    options.candidates = candidates;
    options.use_config_metric = false;
    options.metric = metric;
    options.allow = allow_ids;
    return searchTimed(query, options);
}

std::vector<SearchHit> Engine::search(const std::string& query, int top_k, int candidates) const {
    SearchOptions options = defaultOptions();
    options.top_k = top_k;
    options.candidates = candidates;
    return searchTimed(query, options).hits;
}

std::vector<SearchHit> Engine::search(const std::string& query) const {
    return searchTimed(query, defaultOptions()).hits;
}

std::vector<Candidate> Engine::retrieve(const std::string& query, int k, Metric metric,
                                        const std::vector<int>& allow_ids) const {
    std::vector<float> vector;
    {
        std::lock_guard<std::mutex> lock(mutex_);
        vector = embedder().embed(query);
    }
    return retrieveVectors(vector.data(), static_cast<int>(vector.size()), k, metric, allow_ids);
}

void Engine::addVectors(const std::vector<std::string>& ids, const std::vector<std::string>& texts,
                        const float* vectors, std::int64_t count) {
    std::lock_guard<std::mutex> lock(mutex_);
    if (ids.size() != texts.size()) {
        throw std::invalid_argument("zcgvs: ids and texts must have equal length");
    }
    if (ids.empty()) {
        return;
    }
    if (rescore_store_ != nullptr || lexical_index_ != nullptr) {
        throw std::runtime_error(
            "zcgvs: incremental indexing is unavailable while a rescore store or lexical index is attached; "
            "rebuild those artifacts offline instead");
    }
    corpus_.addDocuments(ids, texts, vectors, count, stream_->get());
}

void Engine::addDocuments(const std::vector<std::string>& ids, const std::vector<std::string>& texts) {
    if (ids.size() != texts.size()) {
        throw std::invalid_argument("zcgvs: ids and texts must have equal length");
    }
    if (ids.empty()) {
        return;
    }
    std::vector<float> vectors;
    {
        std::lock_guard<std::mutex> lock(mutex_);
        const QueryEmbedder& encoder = embedder();
        for (const std::string& text : texts) {
            const std::vector<float> v = encoder.embed(text);
            if (static_cast<int>(v.size()) != corpus_.dim()) {
                throw std::runtime_error("zcgvs: embedding dim mismatch while adding documents");
            }
            vectors.insert(vectors.end(), v.begin(), v.end());
        }
    }
    addVectors(ids, texts, vectors.data(), static_cast<std::int64_t>(ids.size()));
}

EngineStats Engine::stats() const {
    std::lock_guard<std::mutex> lock(mutex_);
    EngineStats s;
    s.corpus_size = corpus_.size();
    s.dim = corpus_.dim();
    s.storage_dtype = scalarName(corpus_.embeddings().dtype());
    s.corpus_bytes = corpus_.embeddings().deviceBytes();
    if (rescore_store_ != nullptr) {
        s.has_rescore_store = true;
        s.rescore_dtype = scalarName(rescore_store_->dtype());
        s.rescore_bytes = rescore_store_->deviceBytes();
    }
    if (lexical_index_ != nullptr) {
        s.has_lexical_index = true;
        s.lexical_postings = lexical_index_->postingCount();
        s.lexical_bytes = lexical_index_->deviceBytes();
    }
    s.has_reranker = false;
    s.graph_captures = searcher_->graphCaptureCount();
    s.graph_launches = searcher_->graphLaunchCount();
    const DeviceInfo info = queryDevice(config_.device_id);
    s.device_name = info.name;
    s.device_total_memory = info.total_memory;
    s.compute_major = info.compute_major;
    s.compute_minor = info.compute_minor;
    return s;
}

}  // namespace zcgvs
