// int8 x int8 MFMA fused scan (per-vector int8 mode): score = (float)(int32 dot) * (s_q * s_r)
// for up to 256 queries per launch against 64-row corpus tiles, with the threshold
// emission of fused.hpp in the epilogue. No counterpart in the reference, whose int8 path is a
// float32 FMA loop (src/cuda/similarity.cu:59-67); this kernel is the batched contraction the
// per-vector int8 configuration needs.
//
// Work split. A workgroup is 8 wavefronts, two per SIMD. Wavefront w keeps the int8 query rows
// of its 32 queries in registers for the whole launch, as v_mfma_i32_32x32x32_i8 B operands
// (query-stationary), so one workgroup covers 256 queries; the two wavefronts of a SIMD hide
// each other's LDS latency and epilogue work behind their MFMAs. Corpus tiles of 64 rows stream through two LDS buffers: while
// the tile in one buffer is multiplied, the next tile's global loads are already in flight into
// registers and are written to the other buffer afterwards, so each corpus byte is read from
// HBM once and from LDS once per wavefront. The A operands of the next K step are read from LDS
// before the MFMAs of the current one are issued, so the LDS latency overlaps the matrix work.
//
// MFMA layout (32x32x32 int8 -> int32, wave64). A (32 x 32, M x K): lane l supplies row l % 32,
// 16 consecutive K values starting at 16 * (l / 32). B (32 x 32, K x N): lane l supplies column
// l % 32 with the same K values. Because A and B use the same K assignment, the product sums
// every dimension exactly once whatever order the hardware walks K in. D: lane l holds column
// l % 32 (the query) and rows 8 * (r / 4) + 4 * (l / 32) + r % 4 for its 16 results r.
//
// LDS tile layout: row r of the tile at r * dim bytes; its 16-byte slot s is stored at slot
// s ^ (r & 7), so the 32 rows one A-operand read touches spread over all banks.
//
// Epilogue of a threshold phase: per lane and query the largest (float)dot * s_r of the tile is
// compared against the query's threshold score with a relative margin of 2^-20 (far above the
// few-ulp difference between that product order and the exact score's), and only when some
// lane of the wavefront passes is the exact score, its key and the key comparison evaluated.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.hpp"
#include "fused.hpp"
#include "scan_core.hpp"

namespace zcgvs_hip {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kRows = kMfmaBlockRows;  // 64 corpus rows per tile
constexpr int kThreads = 512;
constexpr int kQueriesPerLaunch = (kThreads / kWave) * 32;
constexpr int kNB = 1;
constexpr float kFilterMargin = 9.5367431640625e-07f;  // 2^-20

template <int kKSteps, bool kDense>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void mfmaScanKernel(ScanArgs scan, PhaseArgs phase, EmitArgs emit, int q_offset, int q_count) {
    constexpr int kDim = kKSteps * 32;
    constexpr int kSlotsPerRow = kDim / 16;
    constexpr int kTileBytes = kRows * kDim;
    constexpr int kPerThread = kRows * kSlotsPerRow / kThreads;
    static_assert(kRows * kSlotsPerRow % kThreads == 0, "tile slots must split evenly");

    __shared__ __attribute__((aligned(16))) std::uint8_t lds_tile[2][kTileBytes];
    __shared__ __attribute__((aligned(16))) float lds_scale[2][kRows];
    __shared__ std::uint32_t lds_mask[2][kRows / 4];
    __shared__ std::uint32_t lds_count[kQueriesPerLaunch];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int half = lane >> 5;
    const int col = lane & 31;
    const int batch = scan.batch;
    const long long doc_count = scan.doc_count;
    const std::uint8_t* corpus = static_cast<const std::uint8_t*>(scan.corpus);
    const std::int8_t* queries = static_cast<const std::int8_t*>(scan.queries);

    // ---- query fragments and per-lane query constants ----
    const int wave_q0 = wave * 32 * kNB;
    const bool wave_active = wave_q0 < q_count;
    v4i qf[kNB][kKSteps];
    float qscale[kNB];
    std::uint64_t tau[kNB];
    float tau_floor[kNB];
    bool q_valid[kNB];
#pragma unroll
    for (int nb = 0; nb < kNB; ++nb) {
        const int qlocal = wave_q0 + nb * 32 + col;
        q_valid[nb] = qlocal < q_count;
        const int q = q_offset + min(qlocal, q_count - 1);
        const std::int8_t* qrow = queries + static_cast<std::size_t>(q) * kDim + 16 * half;
#pragma unroll
        for (int ks = 0; ks < kKSteps; ++ks) {
            const v4i value = *reinterpret_cast<const v4i*>(qrow + ks * 32);
            qf[nb][ks] = q_valid[nb] ? value : v4i{0, 0, 0, 0};
        }
        qscale[nb] = scan.query_scales[q];
        tau[nb] = 0ull;
        tau_floor[nb] = -INFINITY;
        if constexpr (!kDense) {
            tau[nb] = emit.tau[q];
            if (tau[nb] != 0ull) {
                const float t = keyScore(tau[nb]);
                tau_floor[nb] = t - fabsf(t) * kFilterMargin - 1e-30f;
            }
        }
    }
    for (int i = tid; i < kQueriesPerLaunch; i += kThreads) {
        lds_count[i] = 0u;
    }

    // ---- tile prefetch (global -> registers) and store (registers -> LDS) ----
    uint4 pre[kPerThread];
    float pre_scale = 0.0f;
    std::uint32_t pre_mask = 0xFFFFFFFFu;
    auto prefetch = [&](long long item) {
        const long long row0 = phaseBlock(item, phase.stride, phase.skip) * kRows;
        const std::uint8_t* base = corpus + static_cast<std::size_t>(row0) * kDim;
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const int p = tid + kThreads * i;
            const int r = p / kSlotsPerRow;
            const int s = p - r * kSlotsPerRow;
            pre[i] = row0 + r < doc_count ? loadChunkStreaming(base + r * kDim + s * 16)
                                          : make_uint4(0u, 0u, 0u, 0u);
        }
        if (tid < kRows) {
            const long long row = row0 + tid;
            pre_scale = row < doc_count ? scan.row_scales[row] : 0.0f;
        } else if (tid < kRows + kRows / 4) {
            std::uint32_t word = 0xFFFFFFFFu;
            if (scan.mask != nullptr) {
                word = 0u;
                const long long first = row0 + 4 * (tid - kRows);
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const std::uint32_t allowed =
                        (first + b < doc_count) ? static_cast<std::uint32_t>(scan.mask[first + b]) : 1u;
                    word |= (allowed != 0u ? 0xFFu : 0u) << (8 * b);
                }
            }
            pre_mask = word;
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const int p = tid + kThreads * i;
            const int r = p / kSlotsPerRow;
            const int s = p - r * kSlotsPerRow;
            *reinterpret_cast<uint4*>(&lds_tile[buf][r * kDim + ((s ^ (r & 7)) << 4)]) = pre[i];
        }
        if (tid < kRows) {
            lds_scale[buf][tid] = pre_scale;
        } else if (tid < kRows + kRows / 4) {
            lds_mask[buf][tid - kRows] = pre_mask;
        }
    };

    long long item = blockIdx.x;
    if (item < phase.items) {
        prefetch(item);
        store(0);
    }
    __syncthreads();

    // A-operand LDS offsets: row m = mb * 32 + col, slot 2 * ks + half stored at slot ^ (m & 7).
    const int a_base0 = col * kDim;
    const int a_base1 = (32 + col) * kDim;
    const int swz = col & 7;

    int buf = 0;
    for (; item < phase.items; item += gridDim.x) {
        const long long next = item + gridDim.x;
        if (next < phase.items) {
            prefetch(next);
        }
        const long long row0 = phaseBlock(item, phase.stride, phase.skip) * kRows;

        if (wave_active) {
            v16i acc[2][kNB];
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
                for (int nb = 0; nb < kNB; ++nb) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        acc[mb][nb][r] = 0;
                    }
                }
            }
            const std::uint8_t* tile = lds_tile[buf];
            v4i a_cur0 = *reinterpret_cast<const v4i*>(tile + a_base0 + (((0 + half) ^ swz) << 4));
            v4i a_cur1 = *reinterpret_cast<const v4i*>(tile + a_base1 + (((0 + half) ^ swz) << 4));
#pragma unroll
            for (int ks = 0; ks < kKSteps; ++ks) {
                v4i a_next0 = a_cur0;
                v4i a_next1 = a_cur1;
                if (ks + 1 < kKSteps) {
                    const int slot = ((2 * (ks + 1) + half) ^ swz) << 4;
                    a_next0 = *reinterpret_cast<const v4i*>(tile + a_base0 + slot);
                    a_next1 = *reinterpret_cast<const v4i*>(tile + a_base1 + slot);
                }
#pragma unroll
                for (int nb = 0; nb < kNB; ++nb) {
                    acc[0][nb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_cur0, qf[nb][ks], acc[0][nb], 0, 0, 0);
                    acc[1][nb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_cur1, qf[nb][ks], acc[1][nb], 0, 0, 0);
                }
                a_cur0 = a_next0;
                a_cur1 = a_next1;
            }

            // ---- epilogue ----
            if constexpr (kDense) {
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int rl0 = mb * 32 + 8 * g + 4 * half;
                        const float4 rs = *reinterpret_cast<const float4*>(&lds_scale[buf][rl0]);
                        const std::uint32_t mw = lds_mask[buf][rl0 >> 2];
                        const float rsv[4] = {rs.x, rs.y, rs.z, rs.w};
#pragma unroll
                        for (int nb = 0; nb < kNB; ++nb) {
                            if (!q_valid[nb]) {
                                continue;
                            }
                            const int q = q_offset + wave_q0 + nb * 32 + col;
                            std::uint64_t* dst = emit.dense + static_cast<std::size_t>(q) * emit.dense_stride + item * kRows;
#pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                const long long row = row0 + rl0 + j;
                                const bool allowed = ((mw >> (8 * j)) & 0xFFu) != 0u;
                                const float combined = qscale[nb] * rsv[j];
                                const float score = allowed ? static_cast<float>(acc[mb][nb][4 * g + j]) * combined
                                                            : kMaskedScore;
                                dst[rl0 + j] = row < doc_count ? makeKey(score, static_cast<std::uint32_t>(row)) : 0ull;
                            }
                        }
                    }
                }
            } else {
                // Cheap conservative filter first.
                float best[kNB];
#pragma unroll
                for (int nb = 0; nb < kNB; ++nb) {
                    best[nb] = -INFINITY;
                }
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int rl0 = mb * 32 + 8 * g + 4 * half;
                        const float4 rs = *reinterpret_cast<const float4*>(&lds_scale[buf][rl0]);
                        const std::uint32_t mw = lds_mask[buf][rl0 >> 2];
                        const float rsv[4] = {rs.x, rs.y, rs.z, rs.w};
#pragma unroll
                        for (int nb = 0; nb < kNB; ++nb) {
#pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                const float v = static_cast<float>(acc[mb][nb][4 * g + j]) * rsv[j];
                                const bool allowed = ((mw >> (8 * j)) & 0xFFu) != 0u;
                                best[nb] = fmaxf(best[nb], allowed ? v : kMaskedScore);
                            }
                        }
                    }
                }
                bool pass = false;
#pragma unroll
                for (int nb = 0; nb < kNB; ++nb) {
                    pass = pass || (q_valid[nb] && best[nb] * qscale[nb] >= tau_floor[nb]);
                }
                if (__any(pass)) {
                    // Exact path: evaluate the score exactly as the oracle does and compare keys.
#pragma unroll
                    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
                        for (int g = 0; g < 4; ++g) {
                            const int rl0 = mb * 32 + 8 * g + 4 * half;
                            const float4 rs = *reinterpret_cast<const float4*>(&lds_scale[buf][rl0]);
                            const std::uint32_t mw = lds_mask[buf][rl0 >> 2];
                            const float rsv[4] = {rs.x, rs.y, rs.z, rs.w};
#pragma unroll
                            for (int nb = 0; nb < kNB; ++nb) {
                                const int q = q_offset + wave_q0 + nb * 32 + col;
#pragma unroll
                                for (int j = 0; j < 4; ++j) {
                                    const long long row = row0 + rl0 + j;
                                    const bool allowed = ((mw >> (8 * j)) & 0xFFu) != 0u;
                                    const float combined = qscale[nb] * rsv[j];
                                    const float score = allowed ? static_cast<float>(acc[mb][nb][4 * g + j]) * combined
                                                                : kMaskedScore;
                                    if (q_valid[nb] && row < doc_count && score >= tau_floor[nb]) {
                                        const std::uint64_t key = makeKey(score, static_cast<std::uint32_t>(row));
                                        if (key > tau[nb]) {
                                            appendCandidate(emit, lds_count, q, q_offset, batch, key);
                                        }
                                    }
                                }
                            }
                        }
                    }
                }
            }
        }

        if (next < phase.items) {
            store(buf ^ 1);
        }
        __syncthreads();
        buf ^= 1;
    }

    if constexpr (!kDense) {
        __syncthreads();
        for (int q = tid; q < q_count; q += kThreads) {
            emit.seg_count[static_cast<std::size_t>(blockIdx.x) * batch + q_offset + q] = lds_count[q];
        }
    }
}

template <int kKSteps>
int launchShape(const ScanArgs& scan, const PhaseArgs& phase, const EmitArgs& emit,
                int workgroups, hipStream_t stream) {
    const int per_launch = kQueriesPerLaunch;
    const long long wanted = phase.dense ? std::min<long long>(phase.items, workgroups) : workgroups;
    const dim3 grid(static_cast<unsigned>(std::max(1LL, wanted)));
    for (int q0 = 0; q0 < scan.batch; q0 += per_launch) {
        const int count = std::min(per_launch, scan.batch - q0);
        if (phase.dense) {
            mfmaScanKernel<kKSteps, true><<<grid, kThreads, 0, stream>>>(scan, phase, emit, q0, count);
        } else {
            mfmaScanKernel<kKSteps, false><<<grid, kThreads, 0, stream>>>(scan, phase, emit, q0, count);
        }
        ZCGVS_LAUNCH_CHECK("mfma scan");
    }
    return ZCGVS_OK;
}

}  // namespace

bool mfmaSupported(const ScanArgs& scan) {
    if (scan.dtype != ZCGVS_DTYPE_I8 || scan.row_scales == nullptr || scan.lexical != nullptr) {
        return false;
    }
    if (scan.metric != ZCGVS_METRIC_COSINE && scan.metric != ZCGVS_METRIC_DOT) {
        return false;
    }
    if (!aligned16(scan.corpus) || !aligned16(scan.queries)) {
        return false;
    }
    switch (scan.dim) {
        case 256:
        case 384:
        case 512:
        case 768:
        case 1024:
            return true;
        default:
            return false;
    }
}

int mfmaWorkgroups() { return deviceComputeUnits(); }

int launchMfmaScan(const ScanArgs& scan, const PhaseArgs& phase, const EmitArgs& emit,
                   int workgroups, hipStream_t stream) {
    if (phase.items <= 0) {
        return ZCGVS_OK;
    }
    switch (scan.dim) {
        case 256: return launchShape<8>(scan, phase, emit, workgroups, stream);
        case 384: return launchShape<12>(scan, phase, emit, workgroups, stream);
        case 512: return launchShape<16>(scan, phase, emit, workgroups, stream);
        case 768: return launchShape<24>(scan, phase, emit, workgroups, stream);
        default: return launchShape<32>(scan, phase, emit, workgroups, stream);
    }
}

}  // namespace zcgvs_hip
