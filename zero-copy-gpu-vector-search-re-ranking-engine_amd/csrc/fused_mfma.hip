// int8 x int8 MFMA fused scan (per-vector int8 mode): score = (float)(int32 dot) * (s_q * s_r)
// for up to 256 queries per launch against 64-row corpus tiles, with the threshold emission of
// fused.hpp in the epilogue. No counterpart in the reference, whose int8 path is a float32 FMA
// loop (src/cuda/similarity.cu:59-67); this kernel is the batched contraction the per-vector int8
// configuration needs.
//
// Work split. A workgroup is 8 wavefronts, two per SIMD. Wavefront w keeps the int8 rows of its
// 32 queries in registers for the whole launch, as v_mfma_i32_32x32x32_i8 B operands
// (query-stationary), so one workgroup covers 256 queries; the two wavefronts of a SIMD hide each
// other's LDS latency and epilogue work behind their MFMAs.
//
// Corpus streaming. Tiles of 64 rows go from HBM straight into a ring of LDS buffers with
// global_load_lds_dwordx4 (no staging registers), kDepth - 1 tiles ahead of the one being
// multiplied. Before a tile is used every wavefront waits for its own copies of that tile
// (s_waitcnt vmcnt with the number of copies issued after it) and then meets the others at a
// bare s_barrier; a __syncthreads() would also wait for the copies of the later tiles and drain
// the ring. Each corpus byte is read from HBM once and from LDS once per wavefront.
//
// MFMA layout (32x32x32 int8 -> int32, wave64). A (32 x 32, M x K): lane l supplies row l % 32,
// 16 consecutive K values starting at 16 * (l / 32). B (32 x 32, K x N): lane l supplies column
// l % 32 with the same K values. Because A and B use the same K assignment, the product sums
// every dimension exactly once whatever order the hardware walks K in. D: lane l holds column
// l % 32 (the query) and rows 8 * (r / 4) + 4 * (l / 32) + r % 4 for its 16 results r.
//
// LDS tile layout: row r at r * dim bytes; its 16-byte slot s is stored at slot s ^ (r & 7), so
// the rows one A-operand read touches spread over the banks. The copy instruction writes 64
// consecutive LDS slots, so each lane computes which global 16 bytes belong to its LDS slot.
//
// Row scales ride along inside the same ring slot (16 lanes of one more 16-byte copy per tile;
// keeping every copy inside one LDS object keeps the compiler from waiting on the in-flight
// copies before each LDS read). They come from a workspace copy of the scales padded to whole
// tiles, in which masked and padding rows hold NaN; such a row scores -FLT_MAX.
//
// Epilogue of a threshold phase: per lane the largest (float)dot * s_r of the tile is compared
// with the query's threshold score minus a relative margin of 2^-20 (far above the few-ulp
// difference between that product order and the exact score's); only when some lane passes is
// the exact score, its key and the key comparison evaluated.
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
constexpr int kWaves = kThreads / kWave;
constexpr int kQueriesPerLaunch = kWaves * 32;
constexpr float kFilterMargin = 9.5367431640625e-07f;  // 2^-20
constexpr std::size_t kRingBudget = 150 * 1024;

// LDS byte address of a __shared__ location.
__device__ __forceinline__ std::uint32_t ldsAddress(const void* p) {
    return static_cast<std::uint32_t>(
        reinterpret_cast<std::uintptr_t>((const __attribute__((address_space(3))) void*)p));
}

// One global_load_lds_dwordx4: every active lane copies 16 bytes from `src` to LDS at
// lds_base + 16 * lane. Issued as inline assembly so that the compiler, which cannot tell the
// ring slots apart, does not make every later LDS read wait for all copies in flight; the
// kernel orders the copies itself (vmcnt waits + barriers). M0 carries the LDS base.
__device__ __forceinline__ void copyToLds(const void* src, std::uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(src), "s"(lds_base)
                 : "memory", "m0");
}

// s_waitcnt that waits until at most n vector-memory operations of this wavefront are pending
// (expcnt and lgkmcnt fields at their "no wait" maxima).
__device__ constexpr int vmcntOnly(int n) {
    return (n & 0xF) | (0x7 << 4) | (0xF << 8) | ((n >> 4) << 14);
}

template <int kKSteps, bool kDense>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void mfmaScanKernel(ScanArgs scan, PhaseArgs phase, EmitArgs emit, int q_offset, int q_count) {
    constexpr int kDim = kKSteps * 32;
    constexpr int kSlotsPerRow = kDim / 16;
    constexpr int kTileBytes = kRows * kDim;
    constexpr int kDepth = 3 * kTileBytes <= static_cast<int>(kRingBudget) ? 3 : 2;
    constexpr int kCopies = kRows * kSlotsPerRow / (kWave * kWaves);  // 16-byte copies per lane
    static_assert(kRows * kSlotsPerRow % (kWave * kWaves) == 0, "tile must split over the waves");
    static_assert(kSlotsPerRow % 8 == 0, "swizzle stays inside a row");

    constexpr int kSlotBytes = kTileBytes + kRows * 4;  // tile, then its 64 row scales
    __shared__ __attribute__((aligned(16))) std::uint8_t ring[kDepth][kSlotBytes];
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
    const int qlocal = wave * 32 + col;
    const bool q_valid = qlocal < q_count;
    const bool wave_active = wave * 32 < q_count;
    const int q = q_offset + min(qlocal, q_count - 1);
    v4i qf[kKSteps];
    {
        const std::int8_t* qrow = queries + static_cast<std::size_t>(q) * kDim + 16 * half;
#pragma unroll
        for (int ks = 0; ks < kKSteps; ++ks) {
            const v4i value = *reinterpret_cast<const v4i*>(qrow + ks * 32);
            qf[ks] = q_valid ? value : v4i{0, 0, 0, 0};
        }
    }
    const float qscale = scan.query_scales[q];
    std::uint64_t tau = 0ull;
    float tau_floor = -INFINITY;
    if constexpr (!kDense) {
        tau = emit.tau[q];
        if (tau != 0ull) {
            const float t = keyScore(tau);
            tau_floor = t <= -3.402823466e+38f ? -INFINITY : t - fabsf(t) * kFilterMargin - 1e-30f;
        }
    }
    for (int i = tid; i < kQueriesPerLaunch; i += kThreads) {
        lds_count[i] = 0u;
    }

    // ---- per-lane copy plan: LDS slot P of the tile holds global slot (P % spr) ^ (row & 7) ----
    int copy_row[kCopies];
    int copy_col[kCopies];
#pragma unroll
    for (int i = 0; i < kCopies; ++i) {
        const int p = (wave * kCopies + i) * kWave + lane;
        const int row = p / kSlotsPerRow;
        const int ls = p - row * kSlotsPerRow;
        copy_row[i] = row;
        copy_col[i] = (ls ^ (row & 7)) * 16;
    }
    auto issue = [&](long long item, int slot) {
        const long long row0 = phaseBlock(item, phase.stride, phase.skip) * kRows;
        const int valid_rows = static_cast<int>(min(static_cast<long long>(kRows), doc_count - row0));
        const std::uint8_t* base = corpus + static_cast<std::size_t>(row0) * kDim;
        const std::uint32_t slot_base = ldsAddress(&ring[slot][0]);
#pragma unroll
        for (int i = 0; i < kCopies; ++i) {
            const int row = min(copy_row[i], valid_rows - 1);  // tail rows re-read the last row
            copyToLds(base + row * kDim + copy_col[i],
                      __builtin_amdgcn_readfirstlane(slot_base + (wave * kCopies + i) * kWave * 16));
        }
        if (wave == 0 && lane < kRows / 4) {
            // the padded scale copy makes rows row0 .. row0 + 63 readable for every tile
            copyToLds(scan.row_scales + row0 + 4 * lane,
                      __builtin_amdgcn_readfirstlane(slot_base + kTileBytes));
        }
    };

    // prologue: fill the ring up to depth - 1 tiles
    const long long stride_items = gridDim.x;
    long long item = blockIdx.x;
#pragma unroll
    for (int d = 0; d < kDepth - 1; ++d) {
        const long long ahead = item + d * stride_items;
        if (ahead < phase.items) {
            issue(ahead, d);
        }
    }
    __syncthreads();  // lds_count initialization visible

    const int a_base0 = col * kDim;
    const int a_base1 = (32 + col) * kDim;
    const int swz = col & 7;

    int slot = 0;
    for (; item < phase.items; item += stride_items) {
        // Wait for this wavefront's copies of the current tile: the ones issued after it belong
        // to the (at most kDepth - 2) later tiles already in flight.
        const long long in_flight = min(static_cast<long long>(kDepth - 2),
                                        (phase.items - 1 - item) / stride_items);
        if (in_flight >= 2) {
            __builtin_amdgcn_s_waitcnt(vmcntOnly(2 * kCopies));
        } else if (in_flight == 1) {
            __builtin_amdgcn_s_waitcnt(vmcntOnly(kCopies));
        } else {
            __builtin_amdgcn_s_waitcnt(vmcntOnly(0));
        }
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");  // no LDS access moves above the barrier
        {
            // Refill the buffer every wavefront finished reading before the barrier.
            const long long ahead = item + (kDepth - 1) * stride_items;
            if (ahead < phase.items) {
                issue(ahead, (slot + kDepth - 1) % kDepth);
            }
        }
        const long long row0 = phaseBlock(item, phase.stride, phase.skip) * kRows;

        if (wave_active) {
            v16i acc0 = {};
            v16i acc1 = {};
            const std::uint8_t* tile = ring[slot];
            v4i a_cur0 = *reinterpret_cast<const v4i*>(tile + a_base0 + ((half ^ swz) << 4));
            v4i a_cur1 = *reinterpret_cast<const v4i*>(tile + a_base1 + ((half ^ swz) << 4));
#pragma unroll
            for (int ks = 0; ks < kKSteps; ++ks) {
                v4i a_next0 = a_cur0;
                v4i a_next1 = a_cur1;
                if (ks + 1 < kKSteps) {
                    const int s = ((2 * (ks + 1) + half) ^ swz) << 4;
                    a_next0 = *reinterpret_cast<const v4i*>(tile + a_base0 + s);
                    a_next1 = *reinterpret_cast<const v4i*>(tile + a_base1 + s);
                }
                acc0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_cur0, qf[ks], acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_cur1, qf[ks], acc1, 0, 0, 0);
                a_cur0 = a_next0;
                a_cur1 = a_next1;
            }

            // ---- epilogue ----
            const float* scales = reinterpret_cast<const float*>(tile + kTileBytes);
            if constexpr (kDense) {
                if (q_valid) {
                    std::uint64_t* dst = emit.dense + static_cast<std::size_t>(q) * emit.dense_stride + item * kRows;
#pragma unroll
                    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
                        for (int g = 0; g < 4; ++g) {
                            const int rl0 = mb * 32 + 8 * g + 4 * half;
                            const float4 rs = *reinterpret_cast<const float4*>(scales + rl0);
                            const float rsv[4] = {rs.x, rs.y, rs.z, rs.w};
#pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                const long long row = row0 + rl0 + j;
                                const int dot = mb == 0 ? acc0[4 * g + j] : acc1[4 * g + j];
                                const float combined = qscale * rsv[j];
                                const float score = rsv[j] == rsv[j] ? static_cast<float>(dot) * combined : kMaskedScore;
                                dst[rl0 + j] = row < doc_count ? makeKey(score, static_cast<std::uint32_t>(row)) : 0ull;
                            }
                        }
                    }
                }
            } else {
                float best = -INFINITY;
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int rl0 = mb * 32 + 8 * g + 4 * half;
                        const float4 rs = *reinterpret_cast<const float4*>(scales + rl0);
                        const float rsv[4] = {rs.x, rs.y, rs.z, rs.w};
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const int dot = mb == 0 ? acc0[4 * g + j] : acc1[4 * g + j];
                            best = fmaxf(best, static_cast<float>(dot) * rsv[j]);  // NaN (masked) ignored
                        }
                    }
                }
                const bool pass = q_valid && best * qscale >= tau_floor;
                if (__any(pass)) {
#pragma unroll
                    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
                        for (int g = 0; g < 4; ++g) {
                            const int rl0 = mb * 32 + 8 * g + 4 * half;
                            const float4 rs = *reinterpret_cast<const float4*>(scales + rl0);
                            const float rsv[4] = {rs.x, rs.y, rs.z, rs.w};
#pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                const long long row = row0 + rl0 + j;
                                const int dot = mb == 0 ? acc0[4 * g + j] : acc1[4 * g + j];
                                const float combined = qscale * rsv[j];
                                const float score = rsv[j] == rsv[j] ? static_cast<float>(dot) * combined : kMaskedScore;
                                if (q_valid && row < doc_count && score >= tau_floor) {
                                    const std::uint64_t key = makeKey(score, static_cast<std::uint32_t>(row));
                                    if (key > tau) {
                                        appendCandidate(emit, lds_count, q, q_offset, batch, key);
                                    }
                                }
                            }
                        }
                    }
                }
            }
        }
        slot = (slot + 1) % kDepth;
    }

    if constexpr (!kDense) {
        __syncthreads();
        for (int i = tid; i < q_count; i += kThreads) {
            emit.seg_count[static_cast<std::size_t>(blockIdx.x) * batch + q_offset + i] = lds_count[i];
        }
    }
}

template <int kKSteps>
int launchShape(const ScanArgs& scan, const PhaseArgs& phase, const EmitArgs& emit,
                int workgroups, hipStream_t stream) {
    const long long wanted = phase.dense ? std::min<long long>(phase.items, workgroups) : workgroups;
    const dim3 grid(static_cast<unsigned>(std::max(1LL, wanted)));
    for (int q0 = 0; q0 < scan.batch; q0 += kQueriesPerLaunch) {
        const int count = std::min(kQueriesPerLaunch, scan.batch - q0);
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
    // The kernel reads no mask: the search merges an allow-mask into the row scales first.
    if (scan.dtype != ZCGVS_DTYPE_I8 || scan.row_scales == nullptr || scan.lexical != nullptr ||
        scan.mask != nullptr) {
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
