// VALU fused scan: scores every visited corpus row against the launch's query range and emits
// selection keys (fused.hpp) instead of writing a [batch, N] matrix. Used for float32, float16,
// reference-mode int8 and binary corpora, and for per-vector int8 when the MFMA kernel does not
// apply. Rows are read as in scan_core.hpp (lane groups, 16-byte chunks, streaming loads); each
// row's chunks are decoded once into registers and reused for every staged query.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.hpp"
#include "fused.hpp"
#include "scan_core.hpp"

namespace zcgvs_hip {

namespace {

constexpr int kKindF32 = ZCGVS_DTYPE_F32;
constexpr int kKindF16 = ZCGVS_DTYPE_F16;
constexpr int kKindI8 = ZCGVS_DTYPE_I8;
constexpr int kKindBinary = ZCGVS_DTYPE_BINARY;
constexpr int kKindI8I8 = 4;

constexpr int kMaxChunksPerLane = 8;
// Binary rows are short (at most 16 chunks): a lane holds at most 2 of a row's chunks, and the
// loads of kBinarySets rows per lane are issued before any of them is scored, so a wavefront keeps
// as many bytes in flight as on the longer float rows.
constexpr int kBinaryChunksPerLane = 2;
constexpr int kBinarySets = 4;

__host__ __device__ constexpr int chunksPerLaneOf(int kind) {
    return kind == ZCGVS_DTYPE_BINARY ? kBinaryChunksPerLane : kMaxChunksPerLane;
}
__host__ __device__ constexpr int rowSetsOf(int kind) { return kind == ZCGVS_DTYPE_BINARY ? kBinarySets : 1; }
// At least 8 lanes (128 contiguous bytes) per row: with one lane per short row (binary, small
// int8) every load instruction of a wavefront touched 64 cache lines for 16 bytes each.
constexpr int kMinRowLanes = 8;
constexpr std::size_t kValuQueryLds = 60 * 1024;

int kindOf(const ScanArgs& scan) {
    if (scan.dtype == ZCGVS_DTYPE_I8 && scan.row_scales != nullptr) {
        return kKindI8I8;
    }
    return scan.dtype;
}

// Bytes of one staged query of this kind (chunk-padded).
__host__ __device__ std::size_t queryStageBytes(int kind, int chunks) {
    switch (kind) {
        case kKindBinary:
        case kKindI8I8:
            return static_cast<std::size_t>(chunks) * 16;  // packed words
        case kKindF16:
            return static_cast<std::size_t>(chunks) * 8 * sizeof(float);
        case kKindI8:
            return static_cast<std::size_t>(chunks) * 16 * sizeof(float);
        default:
            return static_cast<std::size_t>(chunks) * 4 * sizeof(float);
    }
}

int chunksOf(const ScanArgs& scan) {
    return static_cast<int>(rowBytes(scan.dtype, scan.dim) / 16);
}

// kTile: queries scored per pass over a row (1 for single-query launches, which then keep one
// accumulator per lane instead of a tile's worth).
template <int kKind, int L, int kTile>
__global__ __launch_bounds__(kScanThreads) void valuScanKernel(ScanArgs scan, PhaseArgs phase,
                                                               EmitArgs emit, int chunks,
                                                               int q_offset, int q_count) {
    extern __shared__ float4 lds_vec[];
    const int stage_words = static_cast<int>(queryStageBytes(kKind, chunks) / 4);
    std::uint32_t* staged = reinterpret_cast<std::uint32_t*>(lds_vec);
    std::uint64_t* lds_tau =
        reinterpret_cast<std::uint64_t*>(staged + static_cast<std::size_t>(q_count) * stage_words);
    std::uint32_t* lds_count = reinterpret_cast<std::uint32_t*>(lds_tau + q_count);
    float* lds_inverse = reinterpret_cast<float*>(lds_count + q_count);
    float* lds_qscale = lds_inverse + q_count;

    const int dim = scan.dim;
    const int batch = scan.batch;
    // ---- stage queries ----
    if constexpr (kKind == kKindBinary) {
        const std::uint32_t* src = static_cast<const std::uint32_t*>(scan.queries);
        const int words = chunks * 4;
        for (int i = threadIdx.x; i < q_count * words; i += blockDim.x) {
            staged[i] = src[static_cast<std::size_t>(q_offset) * words + i];
        }
    } else if constexpr (kKind == kKindI8I8) {
        const std::int8_t* src = static_cast<const std::int8_t*>(scan.queries);
        const int words = chunks * 4;
        for (int i = threadIdx.x; i < q_count * words; i += blockDim.x) {
            const int q = i / words;
            const int w = i - q * words;
            std::uint32_t packed = 0u;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int j = 4 * w + b;
                const int value =
                    j < dim ? static_cast<int>(src[static_cast<std::size_t>(q_offset + q) * dim + j]) : 0;
                packed |= static_cast<std::uint32_t>(value & 0xFF) << (8 * b);
            }
            staged[i] = packed;
        }
    } else {
        const float* src = static_cast<const float*>(scan.queries);
        float* fstaged = reinterpret_cast<float*>(staged);
        for (int i = threadIdx.x; i < q_count * stage_words; i += blockDim.x) {
            const int q = i / stage_words;
            const int j = i - q * stage_words;
            fstaged[i] = j < dim ? src[static_cast<std::size_t>(q_offset + q) * dim + j] : 0.0f;
        }
    }
    for (int q = threadIdx.x; q < q_count; q += blockDim.x) {
        lds_tau[q] = phase.dense ? 0ull : emit.tau[q_offset + q];
        lds_count[q] = 0u;
        float inverse = 0.0f;
        if (scan.lexical != nullptr) {
            const float peak = scan.lexical_max[q_offset + q];
            inverse = peak > 0.0f ? 1.0f / peak : 0.0f;
        }
        lds_inverse[q] = inverse;
        lds_qscale[q] = scan.query_scales != nullptr ? scan.query_scales[q_offset + q] : 1.0f;
    }
    __syncthreads();

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int group = lane % L;
    constexpr int kRowsPerWave = kWave / L;
    constexpr int kRowsPerIter = (kScanThreads / kWave) * kRowsPerWave;
    const int iters = phase.block_rows / kRowsPerIter;
    const std::size_t row_bytes = static_cast<std::size_t>(chunks) * 16;
    const bool l2 = scan.metric == ZCGVS_METRIC_L2;
    const long long doc_count = scan.doc_count;
    const std::uint8_t* corpus = static_cast<const std::uint8_t*>(scan.corpus);

    constexpr int kPerLane = chunksPerLaneOf(kKind);
    constexpr int kSets = rowSetsOf(kKind);
    for (long long item = blockIdx.x; item < phase.items; item += gridDim.x) {
        const long long row0 = phaseBlock(item, phase.stride, phase.skip) * phase.block_rows;
        for (int it0 = 0; it0 < iters; it0 += kSets) {
            // the loads of kSets row sets first (iters is a multiple of kSets)
            uint4 raws[kSets][kPerLane];
#pragma unroll
            for (int set = 0; set < kSets; ++set) {
                const int local = (it0 + set) * kRowsPerIter + wave * kRowsPerWave + lane / L;
                const long long row = row0 + local;
                const bool live = row < doc_count && !(scan.mask != nullptr && scan.mask[row] == 0);
#pragma unroll
                for (int t = 0; t < kPerLane; ++t) {
                    const int c = group + t * L;
                    raws[set][t] = make_uint4(0u, 0u, 0u, 0u);
                    if (live && c < chunks) {
                        raws[set][t] = loadChunkStreaming(corpus + static_cast<std::size_t>(row) * row_bytes +
                                                          static_cast<std::size_t>(c) * 16);
                    }
                }
            }
#pragma unroll
            for (int set = 0; set < kSets; ++set) {
            const int local = (it0 + set) * kRowsPerIter + wave * kRowsPerWave + lane / L;
            const long long row = row0 + local;
            const bool valid = row < doc_count;
            const bool masked = valid && scan.mask != nullptr && scan.mask[row] == 0;
            const bool live = valid && !masked;
            const uint4 (&raw)[kPerLane] = raws[set];
            float row_scale = 1.0f;
            if constexpr (kKind == kKindI8I8) {
                row_scale = live ? scan.row_scales[row] : 0.0f;
            }

            for (int qt = 0; qt < q_count; qt += kTile) {
                const int tile = min(kTile, q_count - qt);
                float score[kTile];
                if constexpr (kKind == kKindBinary || kKind == kKindI8I8) {
                    int acc[kTile];
#pragma unroll
                    for (int q = 0; q < kTile; ++q) {
                        acc[q] = 0;
                    }
#pragma unroll
                    for (int t = 0; t < kPerLane; ++t) {
                        const int c = group + t * L;
                        if (c < chunks) {
#pragma unroll
                            for (int q = 0; q < kTile; ++q) {
                                if (q < tile) {
                                    const uint4 qw = *reinterpret_cast<const uint4*>(
                                        staged + static_cast<std::size_t>(qt + q) * stage_words + 4 * c);
                                    if constexpr (kKind == kKindBinary) {
                                        acc[q] += __popc(raw[t].x ^ qw.x) + __popc(raw[t].y ^ qw.y) +
                                                  __popc(raw[t].z ^ qw.z) + __popc(raw[t].w ^ qw.w);
                                    } else {
                                        int a = acc[q];
                                        a = __builtin_amdgcn_sdot4(static_cast<int>(raw[t].x), static_cast<int>(qw.x), a, false);
                                        a = __builtin_amdgcn_sdot4(static_cast<int>(raw[t].y), static_cast<int>(qw.y), a, false);
                                        a = __builtin_amdgcn_sdot4(static_cast<int>(raw[t].z), static_cast<int>(qw.z), a, false);
                                        a = __builtin_amdgcn_sdot4(static_cast<int>(raw[t].w), static_cast<int>(qw.w), a, false);
                                        acc[q] = a;
                                    }
                                }
                            }
                        }
                    }
#pragma unroll
                    for (int q = 0; q < kTile; ++q) {
                        if (q < tile) {
                            const int total = groupSum<L>(acc[q]);
                            if constexpr (kKind == kKindBinary) {
                                score[q] = static_cast<float>(dim - 2 * total) / static_cast<float>(dim);
                            } else {
                                const float combined = lds_qscale[qt + q] * row_scale;
                                score[q] = static_cast<float>(total) * combined;
                            }
                        }
                    }
                } else {
                    using Traits = ChunkTraits<kKind>;
                    constexpr int E = Traits::kElems;
                    float acc[kTile];
#pragma unroll
                    for (int q = 0; q < kTile; ++q) {
                        acc[q] = 0.0f;
                    }
                    const float* fstaged = reinterpret_cast<const float*>(staged);
#pragma unroll
                    for (int t = 0; t < kPerLane; ++t) {
                        const int c = group + t * L;
                        if (c < chunks) {
                            float v[E];
                            Traits::decode(raw[t], scan.scale, v);
#pragma unroll
                            for (int q = 0; q < kTile; ++q) {
                                if (q < tile) {
                                    const float* qv = fstaged + static_cast<std::size_t>(qt + q) * stage_words + c * E;
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
#pragma unroll
                    for (int q = 0; q < kTile; ++q) {
                        if (q < tile) {
                            const float total = groupSum<L>(acc[q]);
                            score[q] = l2 ? -total : total;
                        }
                    }
                }

                // ---- emit ----
#pragma unroll
                for (int q = 0; q < kTile; ++q) {
                    if (q < tile && (q % L) == group) {
                        const int gq = q_offset + qt + q;
                        std::uint64_t key = 0ull;
                        if (valid) {
                            float value = masked ? kMaskedScore : score[q];
                            if (scan.lexical != nullptr) {
                                const float lex = scan.lexical[static_cast<std::size_t>(gq) * doc_count + row];
                                value = fuseHybrid(value, lex, scan.dense_weight, lds_inverse[qt + q]);
                            }
                            key = makeKey(value, static_cast<std::uint32_t>(row));
                        }
                        if (phase.dense) {
                            const long long slot = item * phase.block_rows + local;
                            emit.dense[static_cast<std::size_t>(gq) * emit.dense_stride + slot] = key;
                        } else if (key > lds_tau[qt + q]) {
                            appendCandidate(emit, lds_count, gq, q_offset, batch, key);
                        }
                    }
                }
            }
            }
        }
    }
    if (!phase.dense) {
        __syncthreads();
        for (int q = threadIdx.x; q < q_count; q += blockDim.x) {
            emit.seg_count[static_cast<std::size_t>(blockIdx.x) * batch + q_offset + q] = lds_count[q];
        }
    }
}

template <int kKind, int kTile>
void launchLanes(int lanes, dim3 grid, std::size_t shared, hipStream_t stream, const ScanArgs& scan,
                 const PhaseArgs& phase, const EmitArgs& emit, int chunks, int q_offset, int q_count) {
    switch (lanes) {
        case 1: valuScanKernel<kKind, 1, kTile><<<grid, kScanThreads, shared, stream>>>(scan, phase, emit, chunks, q_offset, q_count); break;
        case 2: valuScanKernel<kKind, 2, kTile><<<grid, kScanThreads, shared, stream>>>(scan, phase, emit, chunks, q_offset, q_count); break;
        case 4: valuScanKernel<kKind, 4, kTile><<<grid, kScanThreads, shared, stream>>>(scan, phase, emit, chunks, q_offset, q_count); break;
        case 8: valuScanKernel<kKind, 8, kTile><<<grid, kScanThreads, shared, stream>>>(scan, phase, emit, chunks, q_offset, q_count); break;
        case 16: valuScanKernel<kKind, 16, kTile><<<grid, kScanThreads, shared, stream>>>(scan, phase, emit, chunks, q_offset, q_count); break;
        case 32: valuScanKernel<kKind, 32, kTile><<<grid, kScanThreads, shared, stream>>>(scan, phase, emit, chunks, q_offset, q_count); break;
        default: valuScanKernel<kKind, 64, kTile><<<grid, kScanThreads, shared, stream>>>(scan, phase, emit, chunks, q_offset, q_count); break;
    }
}

template <int kKind>
void launchKind(int lanes, dim3 grid, std::size_t shared, hipStream_t stream, const ScanArgs& scan,
                const PhaseArgs& phase, const EmitArgs& emit, int chunks, int q_offset,
                int q_count) {
    if (q_count == 1) {
        launchLanes<kKind, 1>(lanes, grid, shared, stream, scan, phase, emit, chunks, q_offset, q_count);
    } else {
        launchLanes<kKind, kQueryTile>(lanes, grid, shared, stream, scan, phase, emit, chunks, q_offset, q_count);
    }
}

}  // namespace

ValuShape valuShape(const ScanArgs& scan) {
    ValuShape shape;
    const int chunks = chunksOf(scan);
    const int kind_of = kindOf(scan);
    shape.lanes = lanesPerRow(chunks, chunksPerLaneOf(kind_of), kMinRowLanes);
    const int rows_per_iter = (kScanThreads / kWave) * (kWave / shape.lanes);
    shape.block_rows = rows_per_iter * std::max(rowSetsOf(kind_of), 64 / rows_per_iter);
    // 8 workgroups (32 wavefronts) per CU: the kernels of short rows fit 7 wavefronts per SIMD,
    // whose extra loads in flight were worth 6% on binary rows; the rest queue behind them
    shape.workgroups = deviceComputeUnits() * 8;
    const std::size_t per_query = queryStageBytes(kind_of, chunks) + 8 + 4 + 4 + 4;
    int group = static_cast<int>(kValuQueryLds / per_query);
    group = std::max(1, std::min(group, scan.batch));
    if (group < scan.batch && group >= kQueryTile) {
        group -= group % kQueryTile;
    }
    shape.query_group = group;
    return shape;
}

// Whether the VALU fused kernel handles this corpus shape (whole 16-byte chunks, at most
// kMaxChunksPerLane chunks per lane).
bool valuSupported(const ScanArgs& scan) {
    const std::size_t bytes = rowBytes(scan.dtype, scan.dim);
    if (bytes % 16 != 0 || !aligned16(scan.corpus)) {
        return false;
    }
    const int chunks = static_cast<int>(bytes / 16);
    const int per_lane = chunksPerLaneOf(kindOf(scan));
    const int lanes = lanesPerRow(chunks, per_lane, kMinRowLanes);
    return (chunks + lanes - 1) / lanes <= per_lane;
}

int launchValuScan(const ScanArgs& scan, const PhaseArgs& phase, const EmitArgs& emit,
                   int workgroups, hipStream_t stream) {
    if (phase.items <= 0) {
        return ZCGVS_OK;
    }
    const ValuShape shape = valuShape(scan);
    const int chunks = chunksOf(scan);
    const int kind = kindOf(scan);
    // Dense phases need no segments, so they may use fewer workgroups than the plan's count.
    const long long wanted = phase.dense ? std::min<long long>(phase.items, workgroups) : workgroups;
    const dim3 grid(static_cast<unsigned>(std::max(1LL, wanted)));
    for (int q0 = 0; q0 < scan.batch; q0 += shape.query_group) {
        const int count = std::min(shape.query_group, scan.batch - q0);
        const std::size_t shared = static_cast<std::size_t>(count) * (queryStageBytes(kind, chunks) + 8 + 4 + 4 + 4);
        switch (kind) {
            case kKindF16: launchKind<kKindF16>(shape.lanes, grid, shared, stream, scan, phase, emit, chunks, q0, count); break;
            case kKindI8: launchKind<kKindI8>(shape.lanes, grid, shared, stream, scan, phase, emit, chunks, q0, count); break;
            case kKindBinary: launchKind<kKindBinary>(shape.lanes, grid, shared, stream, scan, phase, emit, chunks, q0, count); break;
            case kKindI8I8: launchKind<kKindI8I8>(shape.lanes, grid, shared, stream, scan, phase, emit, chunks, q0, count); break;
            default: launchKind<kKindF32>(shape.lanes, grid, shared, stream, scan, phase, emit, chunks, q0, count); break;
        }
        ZCGVS_LAUNCH_CHECK("fused scan");
    }
    return ZCGVS_OK;
}

}  // namespace zcgvs_hip
