// Composition root (include/zcgvs/engine/engine.hpp:29-106): corpus, optional rescore store and
// lexical index, the Searcher and its stream. Vector queries (searchVectors, retrieveVectors) are
// the native entry; the reference's text-query methods run through an attached QueryEmbedder.
// Calls are serialized by a mutex, so one Engine may be shared by threads.
#pragma once

#include <cstdint>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "zcgvs/core/hip_stream.hpp"
#include "zcgvs/data/corpus.hpp"
#include "zcgvs/data/lexical_index.hpp"
#include "zcgvs/engine/engine_config.hpp"
#include "zcgvs/engine/engine_stats.hpp"
#include "zcgvs/engine/query_embedder.hpp"
#include "zcgvs/engine/search_options.hpp"
#include "zcgvs/engine/search_response.hpp"
#include "zcgvs/search/search_result.hpp"
#include "zcgvs/search/searcher.hpp"

namespace zcgvs {

class Engine {
public:
    // Loads the artifacts named by `config` (embeddings, metadata, rescore store, lexical index).
    explicit Engine(const EngineConfig& config);
    // An engine over in-memory parts (rescore / lexical may be null).
    Engine(const EngineConfig& config, Corpus corpus, std::unique_ptr<EmbeddingStore> rescore,
           std::unique_ptr<LexicalIndex> lexical);
    ~Engine();

    Engine(const Engine&) = delete;
    Engine& operator=(const Engine&) = delete;

    void setQueryEmbedder(std::shared_ptr<const QueryEmbedder> embedder);

    SearchOptions defaultOptions() const;

    // queries: [batch, dim] float32 host rows. terms: optional per-query term ids for the hybrid
    // stage (deduplicated and capped at max_query_terms).
    BatchSearchResponse searchVectors(const float* queries, int batch, int dim, const SearchOptions& options,
                                      const std::vector<std::vector<int>>& terms = {}) const;
    std::vector<Candidate> retrieveVectors(const float* query, int dim, int k, Metric metric,
                                           const std::vector<int>& allow_ids) const;

    // Text queries (need a QueryEmbedder).
    SearchResponse searchTimed(const std::string& query, const SearchOptions& options) const;
    BatchSearchResponse searchBatch(const std::vector<std::string>& queries, const SearchOptions& options) const;
    SearchResponse searchTimed(const std::string& query, int top_k, int candidates, Metric metric,
                               const std::vector<int>& allow_ids) const;
    std::vector<SearchHit> search(const std::string& query, int top_k, int candidates) const;
    std::vector<SearchHit> search(const std::string& query) const;
    std::vector<Candidate> retrieve(const std::string& query, int k, Metric metric,
                                    const std::vector<int>& allow_ids) const;

    void addDocuments(const std::vector<std::string>& ids, const std::vector<std::string>& texts);
    void addVectors(const std::vector<std::string>& ids, const std::vector<std::string>& texts,
                    const float* vectors, std::int64_t count);

    EngineStats stats() const;
    std::int64_t corpusSize() const;
    int dim() const { return corpus_.dim(); }
    std::string storageDtype() const;
    bool hasLexicalIndex() const { return lexical_index_ != nullptr; }
    bool hasRescoreStore() const { return rescore_store_ != nullptr; }
    bool hasReranker() const { return false; }
    bool hasQueryEmbedder() const { return embedder_ != nullptr; }
    const EngineConfig& config() const { return config_; }

private:
    struct Resolved {
        int top_k = 10;
        int candidates = 100;
        Metric metric = Metric::Cosine;
        int rescore_candidates = 0;
        float dense_weight = 1.0f;
        bool hybrid = false;
        bool use_graph = false;
    };

    void attach();
    Resolved resolve(const SearchOptions& options, std::int64_t corpus_size) const;
    const std::uint8_t* buildMask(const std::vector<int>& allow_ids, std::int64_t doc_count) const;
    std::vector<int> dedupeTerms(const std::vector<int>& terms) const;
    BatchSearchResponse runBatch(const float* queries, int batch, const SearchOptions& options,
                                 const std::vector<std::vector<int>>& terms, double embed_ms,
                                 double tokenize_ms) const;
    std::vector<SearchHit> assemble(const HostTopK& selection, int query, const Resolved& resolved) const;
    const QueryEmbedder& embedder() const;

    EngineConfig config_;
    Corpus corpus_;
    std::unique_ptr<EmbeddingStore> rescore_store_;
    std::unique_ptr<LexicalIndex> lexical_index_;
    std::shared_ptr<const QueryEmbedder> embedder_;
    std::unique_ptr<HipStream> stream_;
    std::unique_ptr<Searcher> searcher_;
    mutable std::mutex mutex_;
    mutable std::vector<std::uint8_t> host_mask_;
    mutable DeviceBuffer<std::uint8_t> d_mask_;
    mutable std::vector<int> host_terms_;
};

}  // namespace zcgvs
