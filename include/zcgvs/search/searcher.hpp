// Drives the device search pipeline (include/zcgvs/search/searcher.hpp:32-141) through the C ABI's
// fused entry zcgvs_search_topk: prepared queries -> phased scan with in-kernel selection ->
// optional hybrid fusion and gather rescore -> [batch, k] ids and scores. Owns a grow-only
// workspace, pinned staging and (optionally) an instantiated HIP graph of the pipeline.
//
// Exactness: the fused scan bounds its per-workgroup candidate buffers. A query whose buffers
// overflow (only inputs whose score order defeats the sampling do this) is recomputed by
// copyResultToHost with the reference-order pipeline (ZCGVS_SEARCH_MATERIALIZE), so every
// returned result is exact.
#pragma once

#include <cstdint>
#include <vector>

#include "zcgvs/core/device_buffer.hpp"
#include "zcgvs/core/hip_stream.hpp"
#include "zcgvs/data/embedding_store.hpp"
#include "zcgvs/data/lexical_index.hpp"
#include "zcgvs/search/search_params.hpp"
#include "zcgvs/search/search_result.hpp"

namespace zcgvs {

class Searcher {
public:
    explicit Searcher(const EmbeddingStore& store);
    ~Searcher();

    Searcher(const Searcher&) = delete;
    Searcher& operator=(const Searcher&) = delete;

    // Exact-precision copy of the corpus in the same document order for the rescore stage
    // (nullptr disables it). Must match the corpus dim and must not be binary.
    void setRescoreStore(const EmbeddingStore* store);

    // CSR inverted index for the hybrid stage (nullptr disables it).
    void setLexicalIndex(const LexicalIndex* index);

    // Host float32 queries [batch, dim]; uploaded through pinned staging on `stream`.
    void search(const float* host_queries, int dim, int batch, const SearchParams& params,
                const HipStream& stream);

    // Queries already in device memory [batch, dim] (no upload). They must stay valid until
    // copyResultToHost returns.
    void searchDevice(const float* device_queries, int dim, int batch, const SearchParams& params,
                      const HipStream& stream);

    HostTopK copyResultToHost(const HipStream& stream);

    // Device [batch, k] results of the last search (valid until the next search).
    const int* deviceIndices() const { return d_out_indices_.data(); }
    const float* deviceScores() const { return d_out_values_.data(); }

    int resultK() const { return current_k_; }
    int resultBatch() const { return current_batch_; }
    double lastSearchGpuMs() const { return last_gpu_ms_; }
    bool lastSearchUsedGraph() const { return used_graph_; }
    std::uint64_t graphCaptureCount() const { return graph_captures_; }
    std::uint64_t graphLaunchCount() const { return graph_launches_; }
    // Queries whose result came from the device's exact fallback (candidate buffers overflowed),
    // counted when results are copied to the host.
    std::uint64_t exactRecomputeCount() const { return exact_recomputes_; }

    bool hasRescoreStore() const { return rescore_store_ != nullptr; }
    bool hasLexicalIndex() const { return lexical_index_ != nullptr; }

private:
    struct GraphKey {
        const void* corpus = nullptr;
        const void* row_scales = nullptr;
        const void* rescore_corpus = nullptr;
        const void* lexical_index = nullptr;
        const void* queries = nullptr;
        const std::uint8_t* mask = nullptr;
        std::uint64_t generation = 0;
        std::int64_t doc_count = 0;
        int k = 0;
        int batch = 0;
        int rescore_candidates = 0;
        int lexical_stride = 0;
        int metric = 0;
        float dense_weight = 1.0f;

        bool operator==(const GraphKey& other) const;
    };

    void validate(int dim, int batch, const SearchParams& params, std::int64_t doc_count) const;
    bool rescoreEnabled(const SearchParams& params) const;
    bool lexicalEnabled(const SearchParams& params) const;
    zcgvs_search_desc describe(const float* queries, int batch, const SearchParams& params) const;
    void ensureCapacity(int batch, const SearchParams& params, const zcgvs_search_desc& desc);
    void run(const float* device_queries, int dim, int batch, const SearchParams& params,
             const HipStream& stream);
    void destroyGraph() noexcept;

    const EmbeddingStore& store_;
    const EmbeddingStore* rescore_store_ = nullptr;
    const LexicalIndex* lexical_index_ = nullptr;
    int dim_ = 0;

    DeviceBuffer<float> d_queries_;
    DeviceBuffer<int> d_query_terms_;
    DeviceBuffer<std::uint8_t> d_workspace_;
    DeviceBuffer<int> d_out_indices_;
    DeviceBuffer<float> d_out_values_;
    PinnedBuffer<float> h_queries_;
    PinnedBuffer<int> h_query_terms_;
    PinnedBuffer<int> h_out_indices_;
    PinnedBuffer<float> h_out_values_;
    PinnedBuffer<std::uint32_t> h_overflow_;

    zcgvs_search_desc last_desc_{};
    std::uint64_t generation_ = 0;
    int current_k_ = 0;
    int current_batch_ = 0;

    HipEvent ev_start_;
    HipEvent ev_end_;
    double last_gpu_ms_ = 0.0;

    zcgvs_graph_t graph_ = nullptr;
    GraphKey graph_key_;
    bool used_graph_ = false;
    std::uint64_t graph_captures_ = 0;
    std::uint64_t graph_launches_ = 0;
    std::uint64_t exact_recomputes_ = 0;
};

}  // namespace zcgvs
