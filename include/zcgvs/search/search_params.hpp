// One device-side search request (include/zcgvs/search/search_params.hpp:24-46).
#pragma once

#include <cstdint>

#include "zcgvs/core/metric.hpp"

namespace zcgvs {

// Who computes scores. Custom is this build's kernels; Cublas names the reference's vendor-GEMM
// yardstick, which this build does not carry: requests for it run the Custom path (the reference
// also falls back to Custom whenever cuBLAS cannot serve a request).
enum class SimilarityBackend : std::int32_t {
    Custom = 0,
    Cublas = 1,
};

inline const char* similarityBackendName(SimilarityBackend backend) {
    return backend == SimilarityBackend::Cublas ? "cublas" : "custom";
}

struct SearchParams {
    int k = 10;
    Metric metric = Metric::Cosine;

    // Optional [doc_count] uint8 device allow-mask; masked documents never enter the top-k.
    const std::uint8_t* d_mask = nullptr;

    // With a rescore store attached and this positive, the primary scan keeps this many
    // candidates and an exact-precision gather re-scores them before the final top-k.
    int rescore_candidates = 0;

    // [batch, lexical_stride] host term ids, -1 padded; used when a lexical index is attached and
    // lexical_stride is positive.
    const int* host_query_terms = nullptr;
    int lexical_stride = 0;

    // Weight of the dense score in the hybrid fusion; 1.0 is dense-only.
    float dense_weight = 1.0f;

    SimilarityBackend backend = SimilarityBackend::Custom;
    bool use_graph = false;
};

}  // namespace zcgvs
