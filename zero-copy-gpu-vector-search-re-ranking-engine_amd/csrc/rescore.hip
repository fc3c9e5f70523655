// Candidate gather + exact rescore (src/cuda/rescore.cu:20-63, 83-130) and the index remap
// (src/cuda/rescore.cu:65-79, 132-146).
//
// One wavefront scores one candidate: its lanes read the candidate row with 16-byte loads (or
// element-wise for rows that are not whole chunks) against the float32 query staged in LDS, and
// the partial sums are combined with an xor butterfly. A block of four wavefronts handles
// kCandidatesPerBlock candidates of one query, so the query is staged once per 16 candidates.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.hpp"
#include "rescore.hpp"
#include "scan_core.hpp"

namespace zcgvs_hip {

namespace {

constexpr int kRescoreThreads = 256;
constexpr int kCandidatesPerBlock = 16;
constexpr int kRemapThreads = 256;

template <int kDtype>
__device__ __forceinline__ float scoreRow(const std::uint8_t* row, int dim, int chunks,
                                          bool chunked, float scale, const float* query,
                                          bool l2, int lane) {
    float acc = 0.0f;
    if (chunked) {
        using Traits = ChunkTraits<kDtype>;
        constexpr int E = Traits::kElems;
        for (int c = lane; c < chunks; c += kWave) {
            float v[E];
            Traits::decode(loadChunk(row + static_cast<std::size_t>(c) * 16), scale, v);
            const float* qv = query + c * E;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                if (l2) {
                    const float d = qv[e] - v[e];
                    acc = fmaf(d, d, acc);
                } else {
                    acc = fmaf(qv[e], v[e], acc);
                }
            }
        }
    } else {
        for (int j = lane; j < dim; j += kWave) {
            float x;
            if constexpr (kDtype == ZCGVS_DTYPE_F32) {
                x = reinterpret_cast<const float*>(row)[j];
            } else if constexpr (kDtype == ZCGVS_DTYPE_F16) {
                x = __half2float(reinterpret_cast<const __half*>(row)[j]);
            } else {
                x = static_cast<float>(reinterpret_cast<const std::int8_t*>(row)[j]) * scale;
            }
            if (l2) {
                const float d = query[j] - x;
                acc = fmaf(d, d, acc);
            } else {
                acc = fmaf(query[j], x, acc);
            }
        }
    }
    acc = groupSum<kWave>(acc);
    return l2 ? -acc : acc;
}

// kFromKeys: candidate ids come from 64-bit selection keys (fused search) instead of int ids.
// kToKeys: results are written as selection keys (score, corpus id) instead of float values.
template <int kDtype, bool kFromKeys, bool kToKeys>
__global__ __launch_bounds__(kRescoreThreads) void gatherRescoreKernel(
    const std::uint8_t* __restrict__ corpus, int doc_count, int dim, int chunks, bool chunked,
    float scale, const float* __restrict__ queries, const void* __restrict__ candidates,
    int candidate_count, int metric, void* __restrict__ values) {
    extern __shared__ float4 lds_vec[];
    float* query = reinterpret_cast<float*>(lds_vec);
    const int q = blockIdx.y;
    for (int t = threadIdx.x; t < dim; t += blockDim.x) {
        query[t] = queries[static_cast<std::size_t>(q) * dim + t];
    }
    __syncthreads();
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const bool l2 = metric == ZCGVS_METRIC_L2;
    const std::size_t row_bytes = rowBytes(kDtype, dim);
    for (int i = wave; i < kCandidatesPerBlock; i += kRescoreThreads / kWave) {
        const int slot = blockIdx.x * kCandidatesPerBlock + i;
        if (slot >= candidate_count) {
            break;
        }
        const std::size_t offset = static_cast<std::size_t>(q) * candidate_count + slot;
        int doc;
        if constexpr (kFromKeys) {
            const std::uint64_t key = static_cast<const std::uint64_t*>(candidates)[offset];
            doc = key == 0ull ? -1 : keyIndex(key);
        } else {
            doc = static_cast<const int*>(candidates)[offset];
        }
        const bool valid = doc >= 0 && doc < doc_count;
        float value = kMaskedScore;
        if (valid) {
            value = scoreRow<kDtype>(corpus + static_cast<std::size_t>(doc) * row_bytes, dim,
                                     chunks, chunked, scale, query, l2, lane);
        }
        if (lane == 0) {
            if constexpr (kToKeys) {
                static_cast<std::uint64_t*>(values)[offset] =
                    valid ? makeKey(value, static_cast<std::uint32_t>(doc)) : 0ull;
            } else {
                static_cast<float*>(values)[offset] = value;
            }
        }
    }
}

__global__ void remapIndicesKernel(const int* __restrict__ candidate_indices,
                                   const int* __restrict__ local_indices, int candidate_count,
                                   int k, int* __restrict__ out_indices) {
    const int q = blockIdx.y;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < k; i += gridDim.x * blockDim.x) {
        const std::size_t o = static_cast<std::size_t>(q) * k + i;
        const int local = local_indices[o];
        out_indices[o] = (local >= 0 && local < candidate_count)
                             ? candidate_indices[static_cast<std::size_t>(q) * candidate_count + local]
                             : -1;
    }
}

template <bool kFromKeys, bool kToKeys>
int launchGather(const void* corpus, int dtype, float scale, int doc_count, int dim,
                 const float* queries, int batch, const void* candidates, int candidate_count,
                 int metric, void* values, hipStream_t stream) {
    const std::size_t row_bytes = rowBytes(dtype, dim);
    const bool chunked = row_bytes % 16 == 0 && aligned16(corpus);
    const int chunks = static_cast<int>(row_bytes / 16);
    // The staged query is padded to whole chunks; for chunked rows dim already is.
    const std::size_t shared = static_cast<std::size_t>(dim) * sizeof(float);
    const dim3 grid(static_cast<unsigned>((candidate_count + kCandidatesPerBlock - 1) / kCandidatesPerBlock),
                    static_cast<unsigned>(batch));
    const std::uint8_t* rows = static_cast<const std::uint8_t*>(corpus);
    switch (dtype) {
        case ZCGVS_DTYPE_F16:
            gatherRescoreKernel<ZCGVS_DTYPE_F16, kFromKeys, kToKeys><<<grid, kRescoreThreads, shared, stream>>>(
                rows, doc_count, dim, chunks, chunked, scale, queries, candidates, candidate_count, metric, values);
            break;
        case ZCGVS_DTYPE_I8:
            gatherRescoreKernel<ZCGVS_DTYPE_I8, kFromKeys, kToKeys><<<grid, kRescoreThreads, shared, stream>>>(
                rows, doc_count, dim, chunks, chunked, scale, queries, candidates, candidate_count, metric, values);
            break;
        default:
            gatherRescoreKernel<ZCGVS_DTYPE_F32, kFromKeys, kToKeys><<<grid, kRescoreThreads, shared, stream>>>(
                rows, doc_count, dim, chunks, chunked, scale, queries, candidates, candidate_count, metric, values);
            break;
    }
    ZCGVS_LAUNCH_CHECK("gather rescore");
    return ZCGVS_OK;
}

}  // namespace

int launchRescoreKeys(const void* corpus, int dtype, float scale, int doc_count, int dim,
                      const float* queries, int batch, const std::uint64_t* candidate_keys,
                      int candidate_count, int metric, std::uint64_t* out_keys,
                      hipStream_t stream) {
    return launchGather<true, true>(corpus, dtype, scale, doc_count, dim, queries, batch,
                                    candidate_keys, candidate_count, metric, out_keys, stream);
}

}  // namespace zcgvs_hip

using namespace zcgvs_hip;

extern "C" {

std::size_t zcgvs_rescore_shared_bytes(int dim) {
    return dim > 0 ? static_cast<std::size_t>(dim) * sizeof(float) : 0;
}

int zcgvs_launch_gather_rescore(const void* d_corpus, int dtype, float scale, int doc_count,
                                int dim, const float* d_queries, int batch,
                                const int* d_candidate_indices, int candidate_count, int metric,
                                float* d_values, zcgvs_stream_t stream) {
    if (candidate_count <= 0 || batch <= 0 || dim <= 0) {
        return clearError();
    }
    if (dtype == ZCGVS_DTYPE_BINARY) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT,
                        "zcgvs rescore: the rescore store must hold float32, float16 or int8 rows");
    }
    if (!validDtype(dtype) || !validMetric(metric)) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs rescore: unknown dtype or metric");
    }
    if (d_corpus == nullptr || d_queries == nullptr || d_candidate_indices == nullptr ||
        d_values == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs rescore: null device pointer");
    }
    if (zcgvs_rescore_shared_bytes(dim) > 64 * 1024) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs rescore: embedding dim too large");
    }
    const int status = launchGather<false, false>(d_corpus, dtype, scale, doc_count, dim,
                                                  d_queries, batch, d_candidate_indices,
                                                  candidate_count, metric, d_values,
                                                  toStream(stream));
    return status == ZCGVS_OK ? clearError() : status;
}

int zcgvs_launch_remap_indices(const int* d_candidate_indices, const int* d_local_indices,
                               int candidate_count, int k, int batch, int* d_out_indices,
                               zcgvs_stream_t stream) {
    if (k <= 0 || batch <= 0) {
        return clearError();
    }
    if (d_candidate_indices == nullptr || d_local_indices == nullptr || d_out_indices == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs remap: null device pointer");
    }
    const unsigned blocks = static_cast<unsigned>((k + kRemapThreads - 1) / kRemapThreads);
    remapIndicesKernel<<<dim3(blocks, static_cast<unsigned>(batch)), kRemapThreads, 0,
                         toStream(stream)>>>(d_candidate_indices, d_local_indices,
                                             candidate_count, k, d_out_indices);
    ZCGVS_LAUNCH_CHECK("remap");
    return clearError();
}

}  // extern "C"
