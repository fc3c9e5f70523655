// Materialized similarity scan: zcgvs_launch_similarity (src/cuda/similarity.cu:345-398) and its
// int8 x int8 per-vector-scale sibling. Writes the full [batch, doc_count] score matrix.
//
// One launch covers the whole batch: blockIdx.y selects a tile of up to kQueryTile queries that
// is staged in LDS once per block, and the blocks stride over the corpus. Rows whose size is a
// multiple of 16 bytes (and a 16-byte aligned base) take the chunked path of scan_core.hpp; any
// other shape takes the scalar path (one wavefront per row, lanes stride the elements). Query
// batches that a matrix-core scan takes (float32 / float16 from 4 queries, per-vector int8 from 8;
// cosine or dot, no mask, its dimensions) run that scan in its store form instead: one pass over
// the corpus for up to 128 (float) or 256 (int8) queries, every score written to the matrix. A lane
// holds up to kLoadBatch chunks of its row and issues all their loads before it uses any of them,
// so they are in flight together; the sums take the chunks in column order as before. Float rows
// are read with the streaming hint (each byte is read once per query tile; for int8 rows it
// measured slower). Measured on a
// single-query 1M x 384 scan, against one load at a time with four chunks per lane: float32
// 0.342 -> 0.232 ms, float16 0.186 -> 0.117 ms, int8 0.119 -> 0.077 ms.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.hpp"
#include "fused.hpp"
#include "scan_core.hpp"

namespace zcgvs_hip {

namespace {

constexpr std::size_t kMaxQueryLdsBytes = 64 * 1024;
constexpr int kLoadBatch = 8;  // chunks per lane (the row layout's bound), all loads in flight together

// ---- float / half / int8 (reference mode) chunked path ----------------------------------------
template <int kDtype, int L>
__global__ __launch_bounds__(kScanThreads) void scanStoreKernel(
    const std::uint8_t* __restrict__ corpus, int doc_count, int dim, int chunks, float scale,
    const float* __restrict__ queries, int batch, const std::uint8_t* __restrict__ mask,
    int metric, float* __restrict__ scores) {
    using Traits = ChunkTraits<kDtype>;
    constexpr int E = Traits::kElems;
    extern __shared__ float4 lds_vec[];
    float* staged = reinterpret_cast<float*>(lds_vec);

    const int query_base = blockIdx.y * kQueryTile;
    const int tile = min(kQueryTile, batch - query_base);
    const int padded = chunks * E;
    for (int i = threadIdx.x; i < tile * dim; i += blockDim.x) {
        const int q = i / dim;
        staged[q * padded + (i - q * dim)] =
            queries[static_cast<std::size_t>(query_base) * dim + i];
    }
    __syncthreads();

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int group = lane % L;
    constexpr int kRowsPerWave = kWave / L;
    const int rows_per_block = (kScanThreads / kWave) * kRowsPerWave;
    const int per_lane = (chunks + L - 1) / L;
    const std::size_t row_bytes = static_cast<std::size_t>(chunks) * 16;
    const bool l2 = metric == ZCGVS_METRIC_L2;

    for (long long base = static_cast<long long>(blockIdx.x) * rows_per_block; base < doc_count;
         base += static_cast<long long>(gridDim.x) * rows_per_block) {
        const long long row = base + wave * kRowsPerWave + lane / L;
        const bool valid = row < doc_count;
        const bool masked = valid && mask != nullptr && mask[row] == 0;
        float acc[kQueryTile];
#pragma unroll
        for (int q = 0; q < kQueryTile; ++q) {
            acc[q] = 0.0f;
        }
        if (valid && !masked) {
            const std::uint8_t* row_ptr = corpus + static_cast<std::size_t>(row) * row_bytes;
            for (int t0 = 0; t0 < per_lane; t0 += kLoadBatch) {
                uint4 raw[kLoadBatch];
#pragma unroll
                for (int i = 0; i < kLoadBatch; ++i) {
                    const int c = group + (t0 + i) * L;
                    const std::uint8_t* at = row_ptr + static_cast<std::size_t>(c) * 16;
                    raw[i] = c >= chunks ? make_uint4(0u, 0u, 0u, 0u)
                                         : (kDtype == ZCGVS_DTYPE_I8 ? loadChunk(at) : loadChunkStreaming(at));
                }
#pragma unroll
                for (int i = 0; i < kLoadBatch; ++i) {
                    const int c = group + (t0 + i) * L;
                    if (c >= chunks) {
                        break;
                    }
                    float v[E];
                    Traits::decode(raw[i], scale, v);
                    const float* qcol = staged + c * E;
#pragma unroll
                    for (int q = 0; q < kQueryTile; ++q) {
                        if (q < tile) {
                            const float* qv = qcol + q * padded;
                            if (l2) {
#pragma unroll
                                for (int e = 0; e < E; ++e) {
                                    const float d = qv[e] - v[e];
                                    acc[q] = fmaf(d, d, acc[q]);
                                }
                            } else {
#pragma unroll
                                for (int e = 0; e < E; ++e) {
                                    acc[q] = fmaf(qv[e], v[e], acc[q]);
                                }
                            }
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int q = 0; q < kQueryTile; ++q) {
            acc[q] = groupSum<L>(acc[q]);
        }
        if (valid) {
#pragma unroll
            for (int q = 0; q < kQueryTile; ++q) {
                if (q < tile && (q % L) == group) {
                    const float value = masked ? kMaskedScore : (l2 ? -acc[q] : acc[q]);
                    scores[static_cast<std::size_t>(query_base + q) * doc_count + row] = value;
                }
            }
        }
    }
}

// ---- scalar path for rows that are not a whole number of 16-byte chunks ----------------------
template <int kDtype>
__device__ __forceinline__ float loadScalar(const std::uint8_t* row, int j, float scale) {
    if constexpr (kDtype == ZCGVS_DTYPE_F32) {
        return reinterpret_cast<const float*>(row)[j];
    } else if constexpr (kDtype == ZCGVS_DTYPE_F16) {
        return __half2float(reinterpret_cast<const __half*>(row)[j]);
    } else {
        return static_cast<float>(reinterpret_cast<const std::int8_t*>(row)[j]) * scale;
    }
}

template <int kDtype>
__global__ __launch_bounds__(kScanThreads) void scanScalarKernel(
    const std::uint8_t* __restrict__ corpus, int doc_count, int dim, std::size_t row_bytes,
    float scale, const float* __restrict__ queries, int batch,
    const std::uint8_t* __restrict__ mask, int metric, float* __restrict__ scores) {
    extern __shared__ float4 lds_vec[];
    float* staged = reinterpret_cast<float*>(lds_vec);
    const int query_base = blockIdx.y * kQueryTile;
    const int tile = min(kQueryTile, batch - query_base);
    for (int i = threadIdx.x; i < tile * dim; i += blockDim.x) {
        staged[i] = queries[static_cast<std::size_t>(query_base) * dim + i];
    }
    __syncthreads();
    const int lane = threadIdx.x & (kWave - 1);
    const int waves = kScanThreads / kWave;
    const bool l2 = metric == ZCGVS_METRIC_L2;
    for (long long row = static_cast<long long>(blockIdx.x) * waves + threadIdx.x / kWave;
         row < doc_count; row += static_cast<long long>(gridDim.x) * waves) {
        const bool masked = mask != nullptr && mask[row] == 0;
        float acc[kQueryTile];
#pragma unroll
        for (int q = 0; q < kQueryTile; ++q) {
            acc[q] = 0.0f;
        }
        if (!masked) {
            const std::uint8_t* row_ptr = corpus + static_cast<std::size_t>(row) * row_bytes;
            for (int j = lane; j < dim; j += kWave) {
                const float x = loadScalar<kDtype>(row_ptr, j, scale);
#pragma unroll
                for (int q = 0; q < kQueryTile; ++q) {
                    if (q < tile) {
                        const float qv = staged[q * dim + j];
                        if (l2) {
                            const float d = qv - x;
                            acc[q] = fmaf(d, d, acc[q]);
                        } else {
                            acc[q] = fmaf(qv, x, acc[q]);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int q = 0; q < kQueryTile; ++q) {
            acc[q] = groupSum<kWave>(acc[q]);
        }
        if (lane < tile) {
            float value = 0.0f;
#pragma unroll
            for (int q = 0; q < kQueryTile; ++q) {
                if (q == lane) {
                    value = acc[q];
                }
            }
            value = masked ? kMaskedScore : (l2 ? -value : value);
            scores[static_cast<std::size_t>(query_base + lane) * doc_count + row] = value;
        }
    }
}

// ---- binary (Hamming) ------------------------------------------------------------------------
// Score (dim - 2h) / dim with IEEE division (include/zcgvs/cuda/decode.cuh:45-47).
template <int L>
__global__ __launch_bounds__(kScanThreads) void hammingStoreKernel(
    const std::uint32_t* __restrict__ corpus, int doc_count, int dim, int words,
    const std::uint32_t* __restrict__ queries, int batch, const std::uint8_t* __restrict__ mask,
    float* __restrict__ scores) {
    extern __shared__ float4 lds_vec[];
    std::uint32_t* staged = reinterpret_cast<std::uint32_t*>(lds_vec);
    const int query_base = blockIdx.y * kQueryTile;
    const int tile = min(kQueryTile, batch - query_base);
    for (int i = threadIdx.x; i < tile * words; i += blockDim.x) {
        staged[i] = queries[static_cast<std::size_t>(query_base) * words + i];
    }
    __syncthreads();

    const bool vectorized = (words % 4) == 0;
    const int chunks = vectorized ? words / 4 : words;  // 4-word chunks or single words
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int group = lane % L;
    constexpr int kRowsPerWave = kWave / L;
    const int rows_per_block = (kScanThreads / kWave) * kRowsPerWave;
    for (long long base = static_cast<long long>(blockIdx.x) * rows_per_block; base < doc_count;
         base += static_cast<long long>(gridDim.x) * rows_per_block) {
        const long long row = base + wave * kRowsPerWave + lane / L;
        const bool valid = row < doc_count;
        const bool masked = valid && mask != nullptr && mask[row] == 0;
        int ham[kQueryTile];
#pragma unroll
        for (int q = 0; q < kQueryTile; ++q) {
            ham[q] = 0;
        }
        if (valid && !masked) {
            const std::uint32_t* row_ptr = corpus + static_cast<std::size_t>(row) * words;
            if (vectorized) {
                for (int c0 = group; c0 < chunks; c0 += kLoadBatch * L) {
                    uint4 raw[kLoadBatch];
#pragma unroll
                    for (int i = 0; i < kLoadBatch; ++i) {
                        const int c = c0 + i * L;
                        raw[i] = c < chunks ? *reinterpret_cast<const uint4*>(row_ptr + 4 * c) : make_uint4(0u, 0u, 0u, 0u);
                    }
#pragma unroll
                    for (int i = 0; i < kLoadBatch; ++i) {
                        const int c = c0 + i * L;
                        if (c >= chunks) {
                            break;
                        }
                        const uint4 bits = raw[i];
#pragma unroll
                        for (int q = 0; q < kQueryTile; ++q) {
                            if (q < tile) {
                                const std::uint32_t* qw = staged + q * words + 4 * c;
                                ham[q] += __popc(bits.x ^ qw[0]) + __popc(bits.y ^ qw[1]) +
                                          __popc(bits.z ^ qw[2]) + __popc(bits.w ^ qw[3]);
                            }
                        }
                    }
                }
            } else {
                for (int c = group; c < chunks; c += L) {
                    const std::uint32_t bits = row_ptr[c];
#pragma unroll
                    for (int q = 0; q < kQueryTile; ++q) {
                        if (q < tile) {
                            ham[q] += __popc(bits ^ staged[q * words + c]);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int q = 0; q < kQueryTile; ++q) {
            ham[q] = groupSum<L>(ham[q]);
        }
        if (valid) {
#pragma unroll
            for (int q = 0; q < kQueryTile; ++q) {
                if (q < tile && (q % L) == group) {
                    const float value =
                        masked ? kMaskedScore
                               : static_cast<float>(dim - 2 * ham[q]) / static_cast<float>(dim);
                    scores[static_cast<std::size_t>(query_base + q) * doc_count + row] = value;
                }
            }
        }
    }
}

// ---- int8 x int8 per-vector scale ------------------------------------------------------------
// score = (float)(int32 dot) * (s_q * s_r), evaluated in exactly this order so the CPU oracle
// reproduces it bit for bit. |dot| <= dim * 127^2 stays below 2^24 for dim <= 1040, where the
// int -> float conversion is exact; larger dims round it (identically on both sides).
template <int L>
__global__ __launch_bounds__(kScanThreads) void scanI8I8StoreKernel(
    const std::uint8_t* __restrict__ corpus, const float* __restrict__ row_scales, int doc_count,
    int chunks, const std::int8_t* __restrict__ queries, const float* __restrict__ query_scales,
    int dim, int batch, const std::uint8_t* __restrict__ mask, float* __restrict__ scores) {
    extern __shared__ float4 lds_vec[];
    int* staged = reinterpret_cast<int*>(lds_vec);  // [tile][chunks * 4] packed int8 words
    const int query_base = blockIdx.y * kQueryTile;
    const int tile = min(kQueryTile, batch - query_base);
    const int padded_words = chunks * 4;
    for (int i = threadIdx.x; i < tile * padded_words; i += blockDim.x) {
        const int q = i / padded_words;
        const int w = i - q * padded_words;
        int packed = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int j = 4 * w + b;
            const int value =
                j < dim ? static_cast<int>(
                              queries[static_cast<std::size_t>(query_base + q) * dim + j])
                        : 0;
            packed |= (value & 0xFF) << (8 * b);
        }
        staged[i] = packed;
    }
    __syncthreads();

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int group = lane % L;
    constexpr int kRowsPerWave = kWave / L;
    const int rows_per_block = (kScanThreads / kWave) * kRowsPerWave;
    const std::size_t row_bytes = static_cast<std::size_t>(chunks) * 16;
    for (long long base = static_cast<long long>(blockIdx.x) * rows_per_block; base < doc_count;
         base += static_cast<long long>(gridDim.x) * rows_per_block) {
        const long long row = base + wave * kRowsPerWave + lane / L;
        const bool valid = row < doc_count;
        const bool masked = valid && mask != nullptr && mask[row] == 0;
        int acc[kQueryTile];
#pragma unroll
        for (int q = 0; q < kQueryTile; ++q) {
            acc[q] = 0;
        }
        if (valid && !masked) {
            const std::uint8_t* row_ptr = corpus + static_cast<std::size_t>(row) * row_bytes;
            for (int c0 = group; c0 < chunks; c0 += kLoadBatch * L) {
                uint4 chunk[kLoadBatch];
#pragma unroll
                for (int i = 0; i < kLoadBatch; ++i) {
                    const int c = c0 + i * L;
                    chunk[i] = c < chunks ? loadChunk(row_ptr + static_cast<std::size_t>(c) * 16) : make_uint4(0u, 0u, 0u, 0u);
                }
#pragma unroll
                for (int i = 0; i < kLoadBatch; ++i) {
                    const int c = c0 + i * L;
                    if (c >= chunks) {
                        break;
                    }
                    const uint4 raw = chunk[i];
#pragma unroll
                    for (int q = 0; q < kQueryTile; ++q) {
                        if (q < tile) {
                            const int* qw = staged + q * padded_words + 4 * c;
                            int a = acc[q];
                            a = __builtin_amdgcn_sdot4(static_cast<int>(raw.x), qw[0], a, false);
                            a = __builtin_amdgcn_sdot4(static_cast<int>(raw.y), qw[1], a, false);
                            a = __builtin_amdgcn_sdot4(static_cast<int>(raw.z), qw[2], a, false);
                            a = __builtin_amdgcn_sdot4(static_cast<int>(raw.w), qw[3], a, false);
                            acc[q] = a;
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int q = 0; q < kQueryTile; ++q) {
            acc[q] = groupSum<L>(acc[q]);
        }
        if (valid) {
            const float row_scale = masked ? 0.0f : row_scales[row];
#pragma unroll
            for (int q = 0; q < kQueryTile; ++q) {
                if (q < tile && (q % L) == group) {
                    float value = kMaskedScore;
                    if (!masked) {
                        const float combined = query_scales[query_base + q] * row_scale;
                        value = static_cast<float>(acc[q]) * combined;
                    }
                    scores[static_cast<std::size_t>(query_base + q) * doc_count + row] = value;
                }
            }
        }
    }
}

// Blocks of a launch: one per rows_per_block rows, at most blocks_per_cu per compute unit (the
// blocks then stride over the corpus). Float rows stream best with 4 per CU, int8 rows in the
// reference's matrix-scale mode (more arithmetic per byte) with 16.
unsigned gridBlocks(long long rows, int rows_per_block, int blocks_per_cu = 8) {
    const long long needed = (rows + rows_per_block - 1) / rows_per_block;
    const long long cap = static_cast<long long>(deviceComputeUnits()) * blocks_per_cu;
    return static_cast<unsigned>(std::max(1LL, std::min(needed, cap)));
}

template <int kDtype, int L>
void launchChunked(const void* corpus, int doc_count, int dim, int chunks, float scale,
                   const float* queries, int batch, const std::uint8_t* mask, int metric,
                   float* scores, std::size_t shared, unsigned tiles, hipStream_t stream) {
    const int rows_per_block = (kScanThreads / kWave) * (kWave / L);
    const dim3 grid(gridBlocks(doc_count, rows_per_block, kDtype == ZCGVS_DTYPE_I8 ? 16 : 4), tiles);
    scanStoreKernel<kDtype, L><<<grid, kScanThreads, shared, stream>>>(
        static_cast<const std::uint8_t*>(corpus), doc_count, dim, chunks, scale, queries, batch,
        mask, metric, scores);
}

template <int kDtype>
void dispatchChunked(int lanes, const void* corpus, int doc_count, int dim, int chunks,
                     float scale, const float* queries, int batch, const std::uint8_t* mask,
                     int metric, float* scores, std::size_t shared, unsigned tiles,
                     hipStream_t stream) {
    switch (lanes) {
        case 1: launchChunked<kDtype, 1>(corpus, doc_count, dim, chunks, scale, queries, batch, mask, metric, scores, shared, tiles, stream); break;
        case 2: launchChunked<kDtype, 2>(corpus, doc_count, dim, chunks, scale, queries, batch, mask, metric, scores, shared, tiles, stream); break;
        case 4: launchChunked<kDtype, 4>(corpus, doc_count, dim, chunks, scale, queries, batch, mask, metric, scores, shared, tiles, stream); break;
        case 8: launchChunked<kDtype, 8>(corpus, doc_count, dim, chunks, scale, queries, batch, mask, metric, scores, shared, tiles, stream); break;
        case 16: launchChunked<kDtype, 16>(corpus, doc_count, dim, chunks, scale, queries, batch, mask, metric, scores, shared, tiles, stream); break;
        case 32: launchChunked<kDtype, 32>(corpus, doc_count, dim, chunks, scale, queries, batch, mask, metric, scores, shared, tiles, stream); break;
        default: launchChunked<kDtype, 64>(corpus, doc_count, dim, chunks, scale, queries, batch, mask, metric, scores, shared, tiles, stream); break;
    }
}

template <int L>
void launchHamming(const void* corpus, int doc_count, int dim, int words, const void* queries,
                   int batch, const std::uint8_t* mask, float* scores, std::size_t shared,
                   unsigned tiles, hipStream_t stream) {
    const int rows_per_block = (kScanThreads / kWave) * (kWave / L);
    const dim3 grid(gridBlocks(doc_count, rows_per_block, 4), tiles);
    hammingStoreKernel<L><<<grid, kScanThreads, shared, stream>>>(
        static_cast<const std::uint32_t*>(corpus), doc_count, dim, words,
        static_cast<const std::uint32_t*>(queries), batch, mask, scores);
}

template <int L>
void launchI8I8(const void* corpus, const float* row_scales, int doc_count, int chunks,
                const std::int8_t* queries, const float* query_scales, int dim, int batch,
                const std::uint8_t* mask, float* scores, std::size_t shared, unsigned tiles,
                hipStream_t stream) {
    const int rows_per_block = (kScanThreads / kWave) * (kWave / L);
    const dim3 grid(gridBlocks(doc_count, rows_per_block), tiles);
    scanI8I8StoreKernel<L><<<grid, kScanThreads, shared, stream>>>(
        static_cast<const std::uint8_t*>(corpus), row_scales, doc_count, chunks, queries,
        query_scales, dim, batch, mask, scores);
}

// The score matrix of a query batch by a matrix-core scan in its store form (every row's score,
// no keys), when one takes the shape: returns false, launching nothing, otherwise.
bool storeOnMatrixCores(const ScanArgs& scan, float* scores, hipStream_t stream, int* status) {
    const bool per_vector = scan.dtype == ZCGVS_DTYPE_I8 && scan.row_scales != nullptr;
    if (per_vector) {
        // whole tiles only: without a padded copy, the scan's last tile reads 64 row scales
        if (!mfmaSupported(scan) || scan.doc_count % kMfmaBlockRows != 0) {
            return false;
        }
    } else if (!mfmaFloatSupported(scan)) {
        return false;
    }
    PhaseArgs phase;
    phase.block_rows = per_vector ? kMfmaBlockRows : mfmaFloatBlockRows(scan);
    phase.items = (scan.doc_count + phase.block_rows - 1) / phase.block_rows;
    phase.dense = 1;
    phase.store = 1;
    EmitArgs emit;
    emit.scores = scores;
    const int workgroups = deviceComputeUnits();
    *status = per_vector ? launchMfmaScan(scan, phase, emit, workgroups, stream)
                         : launchMfmaFloatScan(scan, phase, emit, workgroups, stream);
    return true;
}

std::size_t stagingBytes(int dtype, int dim) {
    if (dtype == ZCGVS_DTYPE_BINARY) {
        return binaryWords(dim) * 4;
    }
    // Padded to whole chunks of the storage type, staged as float32.
    const int per_chunk = elementsPerChunk(dtype);
    const std::size_t padded = static_cast<std::size_t>((dim + per_chunk - 1) / per_chunk) * per_chunk;
    return padded * sizeof(float);
}

}  // namespace

}  // namespace zcgvs_hip

using namespace zcgvs_hip;

extern "C" {

int zcgvs_similarity_query_tile(void) { return kQueryTile; }

std::size_t zcgvs_similarity_shared_bytes(int dtype, int dim, int batch) {
    if (batch <= 0 || dim <= 0 || !validDtype(dtype)) {
        return 0;
    }
    return static_cast<std::size_t>(std::min(batch, kQueryTile)) * stagingBytes(dtype, dim);
}

int zcgvs_launch_similarity(const void* d_corpus, int dtype, float scale, int doc_count, int dim,
                            const void* d_queries, int batch, const std::uint8_t* d_mask,
                            int metric, float* d_scores, zcgvs_stream_t stream) {
    if (doc_count <= 0 || batch <= 0 || dim <= 0) {
        return clearError();
    }
    if (!validDtype(dtype)) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs similarity: unknown storage dtype");
    }
    if (!validMetric(metric)) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs similarity: unknown metric");
    }
    if (d_corpus == nullptr || d_queries == nullptr || d_scores == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs similarity: null device pointer");
    }
    const std::size_t shared = zcgvs_similarity_shared_bytes(dtype, dim, batch);
    if (shared > kMaxQueryLdsBytes) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT,
                        "zcgvs similarity: embedding dim " + std::to_string(dim) +
                            " needs more shared memory than a block can stage");
    }
    const hipStream_t s = toStream(stream);
    const unsigned tiles = static_cast<unsigned>((batch + kQueryTile - 1) / kQueryTile);

    if (dtype == ZCGVS_DTYPE_BINARY) {
        const int words = static_cast<int>(binaryWords(dim));
        const bool vectorized = (words % 4) == 0 && aligned16(d_corpus);
        const int chunks = vectorized ? words / 4 : words;
        // Binary rows are short: one lane per row unless a row spans many chunks.
        const int lanes = vectorized ? lanesPerRow(chunks, kLoadBatch) : 1;
        switch (lanes) {
            case 1: launchHamming<1>(d_corpus, doc_count, dim, words, d_queries, batch, d_mask, d_scores, shared, tiles, s); break;
            case 2: launchHamming<2>(d_corpus, doc_count, dim, words, d_queries, batch, d_mask, d_scores, shared, tiles, s); break;
            case 4: launchHamming<4>(d_corpus, doc_count, dim, words, d_queries, batch, d_mask, d_scores, shared, tiles, s); break;
            case 8: launchHamming<8>(d_corpus, doc_count, dim, words, d_queries, batch, d_mask, d_scores, shared, tiles, s); break;
            case 16: launchHamming<16>(d_corpus, doc_count, dim, words, d_queries, batch, d_mask, d_scores, shared, tiles, s); break;
            case 32: launchHamming<32>(d_corpus, doc_count, dim, words, d_queries, batch, d_mask, d_scores, shared, tiles, s); break;
            default: launchHamming<64>(d_corpus, doc_count, dim, words, d_queries, batch, d_mask, d_scores, shared, tiles, s); break;
        }
        ZCGVS_LAUNCH_CHECK("hamming scan");
        return clearError();
    }

    const std::size_t row_bytes = rowBytes(dtype, dim);
    const float* queries = static_cast<const float*>(d_queries);
    if (dtype != ZCGVS_DTYPE_I8 && d_mask == nullptr) {
        ScanArgs scan;
        scan.corpus = d_corpus;
        scan.doc_count = doc_count;
        scan.dim = dim;
        scan.dtype = dtype;
        scan.scale = scale;
        scan.queries = d_queries;
        scan.batch = batch;
        scan.metric = metric;
        int status = ZCGVS_OK;
        if (storeOnMatrixCores(scan, d_scores, s, &status)) {
            return status == ZCGVS_OK ? clearError() : status;
        }
    }
    if (row_bytes % 16 == 0 && aligned16(d_corpus)) {
        const int chunks = static_cast<int>(row_bytes / 16);
        const int lanes = lanesPerRow(chunks, kLoadBatch);
        switch (dtype) {
            case ZCGVS_DTYPE_F16:
                dispatchChunked<ZCGVS_DTYPE_F16>(lanes, d_corpus, doc_count, dim, chunks, scale, queries, batch, d_mask, metric, d_scores, shared, tiles, s);
                break;
            case ZCGVS_DTYPE_I8:
                dispatchChunked<ZCGVS_DTYPE_I8>(lanes, d_corpus, doc_count, dim, chunks, scale, queries, batch, d_mask, metric, d_scores, shared, tiles, s);
                break;
            default:
                dispatchChunked<ZCGVS_DTYPE_F32>(lanes, d_corpus, doc_count, dim, chunks, scale, queries, batch, d_mask, metric, d_scores, shared, tiles, s);
                break;
        }
    } else {
        const std::size_t scalar_shared =
            static_cast<std::size_t>(std::min(batch, kQueryTile)) * dim * sizeof(float);
        const dim3 grid(gridBlocks(doc_count, kScanThreads / kWave), tiles);
        const std::uint8_t* corpus = static_cast<const std::uint8_t*>(d_corpus);
        switch (dtype) {
            case ZCGVS_DTYPE_F16:
                scanScalarKernel<ZCGVS_DTYPE_F16><<<grid, kScanThreads, scalar_shared, s>>>(corpus, doc_count, dim, row_bytes, scale, queries, batch, d_mask, metric, d_scores);
                break;
            case ZCGVS_DTYPE_I8:
                scanScalarKernel<ZCGVS_DTYPE_I8><<<grid, kScanThreads, scalar_shared, s>>>(corpus, doc_count, dim, row_bytes, scale, queries, batch, d_mask, metric, d_scores);
                break;
            default:
                scanScalarKernel<ZCGVS_DTYPE_F32><<<grid, kScanThreads, scalar_shared, s>>>(corpus, doc_count, dim, row_bytes, scale, queries, batch, d_mask, metric, d_scores);
                break;
        }
    }
    ZCGVS_LAUNCH_CHECK("similarity scan");
    return clearError();
}

int zcgvs_launch_similarity_i8i8(const std::int8_t* d_corpus, const float* d_row_scales,
                                 int doc_count, int dim, const std::int8_t* d_queries,
                                 const float* d_query_scales, int batch,
                                 const std::uint8_t* d_mask, int metric, float* d_scores,
                                 zcgvs_stream_t stream) {
    if (doc_count <= 0 || batch <= 0 || dim <= 0) {
        return clearError();
    }
    if (metric != ZCGVS_METRIC_COSINE && metric != ZCGVS_METRIC_DOT) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT,
                        "zcgvs similarity: int8 x int8 scoring supports cosine and dot only");
    }
    if (d_corpus == nullptr || d_row_scales == nullptr || d_queries == nullptr ||
        d_query_scales == nullptr || d_scores == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs similarity: null device pointer");
    }
    if (dim % 16 != 0 || !aligned16(d_corpus)) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT,
                        "zcgvs similarity: int8 x int8 scoring needs dim % 16 == 0 and a "
                        "16-byte aligned corpus");
    }
    const int chunks = dim / 16;
    const std::size_t shared =
        static_cast<std::size_t>(std::min(batch, kQueryTile)) * chunks * 16;
    if (shared > kMaxQueryLdsBytes) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs similarity: embedding dim too large");
    }
    const unsigned tiles = static_cast<unsigned>((batch + kQueryTile - 1) / kQueryTile);
    const hipStream_t s = toStream(stream);
    if (d_mask == nullptr) {
        ScanArgs scan;
        scan.corpus = d_corpus;
        scan.doc_count = doc_count;
        scan.dim = dim;
        scan.dtype = ZCGVS_DTYPE_I8;
        scan.row_scales = d_row_scales;
        scan.queries = d_queries;
        scan.query_scales = d_query_scales;
        scan.batch = batch;
        scan.metric = metric;
        int status = ZCGVS_OK;
        if (storeOnMatrixCores(scan, d_scores, s, &status)) {
            return status == ZCGVS_OK ? clearError() : status;
        }
    }
    switch (lanesPerRow(chunks, kLoadBatch)) {
        case 1: launchI8I8<1>(d_corpus, d_row_scales, doc_count, chunks, d_queries, d_query_scales, dim, batch, d_mask, d_scores, shared, tiles, s); break;
        case 2: launchI8I8<2>(d_corpus, d_row_scales, doc_count, chunks, d_queries, d_query_scales, dim, batch, d_mask, d_scores, shared, tiles, s); break;
        case 4: launchI8I8<4>(d_corpus, d_row_scales, doc_count, chunks, d_queries, d_query_scales, dim, batch, d_mask, d_scores, shared, tiles, s); break;
        case 8: launchI8I8<8>(d_corpus, d_row_scales, doc_count, chunks, d_queries, d_query_scales, dim, batch, d_mask, d_scores, shared, tiles, s); break;
        case 16: launchI8I8<16>(d_corpus, d_row_scales, doc_count, chunks, d_queries, d_query_scales, dim, batch, d_mask, d_scores, shared, tiles, s); break;
        case 32: launchI8I8<32>(d_corpus, d_row_scales, doc_count, chunks, d_queries, d_query_scales, dim, batch, d_mask, d_scores, shared, tiles, s); break;
        default: launchI8I8<64>(d_corpus, d_row_scales, doc_count, chunks, d_queries, d_query_scales, dim, batch, d_mask, d_scores, shared, tiles, s); break;
    }
    ZCGVS_LAUNCH_CHECK("int8 x int8 scan");
    return clearError();
}

}  // extern "C"
