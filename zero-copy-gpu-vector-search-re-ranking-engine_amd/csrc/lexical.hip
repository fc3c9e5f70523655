// Hybrid lexical stage: BM25 over CSR postings (src/cuda/lexical.cu:17-42, 227-241), the
// per-query positive maximum (lexical.cu:44-65, 243-254) and the convex fusion with the dense
// score (lexical.cu:67-74, 256-272).
//
// Determinism. The reference launches one block per query term and scatter-adds with float
// atomics, so a document hit by several terms sums them in a run-dependent order. Here the term
// slots of a query are processed one launch at a time, in slot order; inside a launch the
// postings of one term touch distinct documents (the index builder emits one posting per
// (term, document)), so every document's sum is ((w_0 + w_1) + w_2) ... in slot order, the order
// of the CPU loop in tests/cpp/test_lexical.cu:71-80, on every run.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.hpp"
#include "rescore.hpp"

namespace zcgvs_hip {

namespace {

constexpr int kPostingThreads = 256;
constexpr int kReduceThreads = 256;

// Postings of term slot `slot` for each query (blockIdx.y) of the batch.
__global__ __launch_bounds__(kPostingThreads) void bm25SlotKernel(
    const std::int64_t* __restrict__ offsets, const int* __restrict__ docs,
    const float* __restrict__ weights, const int* __restrict__ query_terms, int term_stride,
    int slot, int doc_count, int vocab_size, float* __restrict__ scores) {
    const int q = blockIdx.y;
    const int term = query_terms[static_cast<std::size_t>(q) * term_stride + slot];
    if (term < 0 || term >= vocab_size) {
        return;
    }
    const std::int64_t begin = offsets[term];
    const std::int64_t end = offsets[term + 1];
    float* row = scores + static_cast<std::size_t>(q) * doc_count;
    for (std::int64_t p = begin + static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
         p < end; p += static_cast<std::int64_t>(gridDim.x) * blockDim.x) {
        const int doc = docs[p];
        if (doc >= 0 && doc < doc_count) {
            atomicAdd(&row[doc], weights[p]);
        }
    }
}

// max(0, max_i values[q][i]) folded into out_max[q] with an unsigned max on the float bits,
// which orders non-negative floats correctly (lexical.cu:61-63).
__global__ __launch_bounds__(kReduceThreads) void maxPositiveKernel(
    const float* __restrict__ values, int count, float* __restrict__ out_max) {
    __shared__ float partial[kReduceThreads / kWave];
    const int q = blockIdx.y;
    const float* row = values + static_cast<std::size_t>(q) * count;
    float best = 0.0f;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += gridDim.x * blockDim.x) {
        best = fmaxf(best, row[i]);
    }
#pragma unroll
    for (int offset = kWave / 2; offset > 0; offset >>= 1) {
        best = fmaxf(best, waveXor(best, offset));
    }
    if ((threadIdx.x & (kWave - 1)) == 0) {
        partial[threadIdx.x / kWave] = best;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float block_best = 0.0f;
        for (int w = 0; w < kReduceThreads / kWave; ++w) {
            block_best = fmaxf(block_best, partial[w]);
        }
        atomicMax(reinterpret_cast<unsigned int*>(out_max + q), __float_as_uint(block_best));
    }
}

// dense = w * dense + (1 - w) * lexical * inverse, with inverse = 1/max or 0, evaluated as
// separate IEEE multiplies and adds in the reference's operand order.
__global__ __launch_bounds__(kReduceThreads) void fuseScoresKernel(
    float* __restrict__ dense, const float* __restrict__ lexical,
    const float* __restrict__ lexical_max, float weight, int count) {
#pragma clang fp contract(off)
    const float peak = *lexical_max;
    const float inverse = (peak > 0.0f) ? (1.0f / peak) : 0.0f;
    const float lexical_weight = 1.0f - weight;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += gridDim.x * blockDim.x) {
        const float a = weight * dense[i];
        const float b = lexical_weight * lexical[i];
        const float c = b * inverse;
        dense[i] = a + c;
    }
}

__global__ void zeroKernel(float* __restrict__ dst, std::size_t count) {
    const std::size_t stride = static_cast<std::size_t>(gridDim.x) * blockDim.x;
    for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
         i < count; i += stride) {
        dst[i] = 0.0f;
    }
}

unsigned reduceBlocks(long long count) {
    long long blocks = (count + kReduceThreads - 1) / kReduceThreads;
    return static_cast<unsigned>(std::max(1LL, std::min(blocks, 256LL)));
}

unsigned postingBlocks() { return static_cast<unsigned>(std::max(1, deviceComputeUnits())); }

}  // namespace

int launchLexicalScores(const std::int64_t* offsets, const int* docs, const float* weights,
                        int vocab_size, const int* query_terms, int term_stride, int batch,
                        int doc_count, float* lexical, float* lexical_max, hipStream_t stream) {
    const std::size_t elements = static_cast<std::size_t>(batch) * doc_count;
    zeroKernel<<<std::min<std::size_t>(8192, (elements + 255) / 256), 256, 0, stream>>>(lexical, elements);
    zeroKernel<<<1, 256, 0, stream>>>(lexical_max, static_cast<std::size_t>(batch));
    ZCGVS_LAUNCH_CHECK("lexical zero");
    const dim3 grid(postingBlocks(), static_cast<unsigned>(batch));
    for (int slot = 0; slot < term_stride; ++slot) {
        bm25SlotKernel<<<grid, kPostingThreads, 0, stream>>>(offsets, docs, weights, query_terms,
                                                             term_stride, slot, doc_count,
                                                             vocab_size, lexical);
    }
    ZCGVS_LAUNCH_CHECK("bm25");
    maxPositiveKernel<<<dim3(reduceBlocks(doc_count), static_cast<unsigned>(batch)),
                        kReduceThreads, 0, stream>>>(lexical, doc_count, lexical_max);
    ZCGVS_LAUNCH_CHECK("lexical max");
    return ZCGVS_OK;
}

}  // namespace zcgvs_hip

using namespace zcgvs_hip;

extern "C" {

int zcgvs_launch_bm25(const std::int64_t* d_offsets, const int* d_docs, const float* d_weights,
                      const int* d_query_terms, int term_count, int doc_count, float* d_scores,
                      zcgvs_stream_t stream) {
    if (term_count <= 0 || doc_count <= 0) {
        return clearError();
    }
    return zcgvs_launch_bm25_batched(d_offsets, d_docs, d_weights, d_query_terms, term_count, 1,
                                     doc_count, d_scores, stream);
}

int zcgvs_launch_bm25_batched(const std::int64_t* d_offsets, const int* d_docs,
                              const float* d_weights, const int* d_query_terms, int term_stride,
                              int batch, int doc_count, float* d_scores, zcgvs_stream_t stream) {
    if (term_stride <= 0 || doc_count <= 0 || batch <= 0) {
        return clearError();
    }
    if (d_offsets == nullptr || d_query_terms == nullptr || d_scores == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs bm25: null device pointer");
    }
    const dim3 grid(postingBlocks(), static_cast<unsigned>(batch));
    for (int slot = 0; slot < term_stride; ++slot) {
        bm25SlotKernel<<<grid, kPostingThreads, 0, toStream(stream)>>>(
            d_offsets, d_docs, d_weights, d_query_terms, term_stride, slot, doc_count, INT32_MAX,
            d_scores);
    }
    ZCGVS_LAUNCH_CHECK("bm25");
    return clearError();
}

int zcgvs_launch_max_positive(const float* d_values, int count, float* d_max,
                              zcgvs_stream_t stream) {
    if (count <= 0) {
        return clearError();
    }
    if (d_values == nullptr || d_max == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs max: null device pointer");
    }
    maxPositiveKernel<<<dim3(reduceBlocks(count), 1), kReduceThreads, 0, toStream(stream)>>>(
        d_values, count, d_max);
    ZCGVS_LAUNCH_CHECK("max positive");
    return clearError();
}

int zcgvs_launch_fuse_scores(float* d_dense, const float* d_lexical, const float* d_lexical_max,
                             float weight, int count, zcgvs_stream_t stream) {
    if (count <= 0) {
        return clearError();
    }
    if (d_dense == nullptr || d_lexical == nullptr || d_lexical_max == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs fuse: null device pointer");
    }
    fuseScoresKernel<<<reduceBlocks(count), kReduceThreads, 0, toStream(stream)>>>(
        d_dense, d_lexical, d_lexical_max, weight, count);
    ZCGVS_LAUNCH_CHECK("fuse");
    return clearError();
}

}  // extern "C"
