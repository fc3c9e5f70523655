// int8 x int8 MFMA fused scan (per-vector int8 mode): score = (float)(int32 dot) * (s_q * s_r)
// for up to 256 queries per launch against 64-row corpus tiles, with the threshold emission of
// fused.hpp in the epilogue. No counterpart in the reference, whose int8 path is a float32 FMA
// loop (src/cuda/similarity.cu:59-67); this kernel is the batched contraction the per-vector int8
// configuration needs.
//
// Work split. A workgroup is 8 wavefronts, two per SIMD. Wavefront w keeps the int8 rows of its
// 32 queries in registers for the whole launch, as v_mfma_i32_32x32x32_i8 B operands
// (query-stationary), so one workgroup covers 256 queries.
//
// Skew. Of the two wavefronts of a SIMD (chosen at start-up from the hardware SIMD id) one leads
// and one lags: after the tile barrier the leader multiplies tile t and then filters it, while
// the lagger first filters tile t - 1 and then multiplies tile t. So each wavefront's VALU filter
// work runs while the other keeps the SIMD's matrix core busy. The two roles run separate loops,
// so a value one role keeps across the barrier takes no register in the other's multiply. A
// filter that passes owes an exact pass over the row groups it marked; the lagger runs it right
// after its filter, the leader right after the next barrier, both before that step's tile copies
// are issued (its keys go to an LDS staging buffer, so in the loop global stores, which would
// queue behind the copies in the vmcnt order, happen only when that buffer is full). The leader
// issues its share of the tile copies after its multiply, the lagger before its own, so neither
// role's copy issue delays the first MFMAs after the barrier.
//
// Modes. A threshold phase emits the keys above each query's threshold; a dense phase writes
// every key to its fixed slot; a sketch phase emits nothing and records, per slot (a row half of
// a workgroup's lanes), the best exact score of each query. A rerun (EmitArgs::q_list) scans only
// the listed queries, with the segment layout the list defines.
//
// Candidate staging. A query's candidates in a workgroup come from exactly two lanes (its two
// row halves), so each lane owns a candidate segment (segment 2 * workgroup + half) and counts
// its slots in a register: no LDS atomic, and no wait for one's return, on the emission path. A
// key the exact pass accepts is parked in a per-wavefront LDS buffer at a position handed out by
// a wave-wide ballot prefix count; the buffers are written to the segments after the scan loop.
// A global store inside the loop would enter the same in-order vmcnt queue as the tile copies,
// and the next tile wait would have to wait for the store's completion too; only a wavefront
// whose buffer is full stores directly.
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
// LDS tile layout: row r at r * dim bytes; its 16-byte slot s is stored at slot s ^ swizzle(r).
// The LDS serves 64 banks x 4 bytes per clock, and ds_read_b128 serves 16 lanes at a time; the 16
// lanes of one A-operand read hit 16 consecutive rows at the same slot, so swizzle(r) must send
// those rows to 16 different 16-byte bank groups: r & 15 when a row is a whole number of bank
// periods (dim % 256 == 0), (r >> 1) & 7 when it is an odd number of half periods (dim 384). A
// swizzle of r & 7 leaves a 2-way conflict that halves the read rate. The copy instruction writes
// 64 consecutive LDS slots, so each lane computes which global 16 bytes belong to its LDS slot.
//
// Row scales travel in a ring of their own, one deeper than the tile ring, so the scales of tile
// t - 1 stay readable through step t. Full tiles read the caller's scales; with an allow-mask,
// or for the partial last tile, they come from a workspace copy in which masked and padding
// rows hold NaN; such a row scores -FLT_MAX.
//
// Filter of a threshold phase: per lane and group of four rows the largest (float)dot * s_r is
// compared with the query's threshold score minus a relative margin of 2^-20 (far above the
// few-ulp difference between that product order and the exact score's); only for the groups in
// which some lane passes are the exact scores, their keys and the key comparisons evaluated.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.hpp"
#include "fused.hpp"
#include "lds_copy.hpp"
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
constexpr int kStaged = 64;  // candidates parked per wavefront before they reach the segments
constexpr int kMinBatch = 8;

// kMode: kThreshold (emit keys above the threshold), kDense (every key to its fixed slot),
// kSketch (per slot the best exact score, no keys) or kRerun (kThreshold over the queries of
// EmitArgs::q_list; a kernel of its own, so profiles tell the fallback's launches apart).
constexpr int kThreshold = 0;
constexpr int kDenseMode = 1;
constexpr int kSketchMode = 2;
constexpr int kRerunMode = 3;
constexpr int kStoreMode = 4;  // dense, writing float scores (the launcher's score matrix)

template <int kKSteps, int kMode>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void mfmaScanKernel(ScanArgs scan, PhaseArgs phase, EmitArgs emit, int q_offset, int q_count) {
    constexpr bool kStore = kMode == kStoreMode;
    constexpr bool kDense = kMode == kDenseMode || kStore;
    constexpr bool kSketch = kMode == kSketchMode;
    constexpr bool kListed = kMode == kRerunMode;
    constexpr bool kEmits = kMode == kThreshold || kListed;  // keys above a threshold
    constexpr int kDim = kKSteps * 32;
    constexpr int kSlotsPerRow = kDim / 16;
    constexpr int kTileBytes = kRows * kDim;
    constexpr int kDepth = 3 * kTileBytes <= static_cast<int>(kRingBudget) ? 3 : 2;
    constexpr int kScaleDepth = kDepth + 1;
    constexpr int kCopies = kRows * kSlotsPerRow / (kWave * kWaves);  // 16-byte copies per lane
    static_assert(kRows * kSlotsPerRow % (kWave * kWaves) == 0, "tile must split over the waves");
    static_assert(kSlotsPerRow % 8 == 0, "swizzle stays inside a row");
    // swizzle period in slots (the swizzle permutes slots inside aligned groups of this size)
    constexpr int kSwzSlots = kSlotsPerRow % 16 == 0 ? 16 : 8;
    auto swizzle = [](int row) {
        return kSlotsPerRow % 16 == 0 ? (row & 15) : (kSlotsPerRow % 16 == 8 ? ((row >> 1) & 7) : (row & 7));
    };
    static_assert(2 * (kCopies + 1) < 64, "copies in flight fit the vmcnt counter");

    __shared__ __attribute__((aligned(16))) std::uint8_t ring[kDepth][kTileBytes];
    __shared__ __attribute__((aligned(16))) float scale_ring[kScaleDepth][kRows];
    __shared__ std::uint32_t lds_simd[4];
    __shared__ std::uint64_t stage_key[kEmits ? kWaves : 1][kStaged];
    // (segment slot << 9) | (half << 8) | local query
    __shared__ std::uint32_t stage_slot[kEmits ? kWaves : 1][kStaged];

    // A rerun scans list entries [q_offset, q_offset + 256) of q_list; F = *q_list_count entries
    // exist, so a launch past them has nothing to do (uniform over the workgroup).
    int seg_batch = scan.batch;     // query rows of the segment layout
    int seg_log2 = emit.seg_log2;   // slots per segment row
    if constexpr (kListed) {
        const int entries = static_cast<int>(__builtin_amdgcn_readfirstlane(*emit.q_list_count));
        if (entries <= q_offset) {
            return;
        }
        q_count = min(q_count, entries - q_offset);
        seg_batch = entries;
        seg_log2 = rerunSegLog2(emit.seg_log2, scan.batch, entries);
    }

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // wave-uniform: scalar indexing
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
    // entry: the lane's row of the segment layout; q: its query
    const int entry = q_offset + min(qlocal, q_count - 1);
    const int q = kListed ? static_cast<int>(emit.q_list[entry]) : entry;
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
    if constexpr (kEmits) {
        tau = emit.tau[q];
        if (tau != 0ull) {
            const float t = keyScore(tau);
            tau_floor = t <= -3.402823466e+38f ? -INFINITY : t - fabsf(t) * kFilterMargin - 1e-30f;
        }
    }
    if (tid < 4) {
        lds_simd[tid] = 0u;
    }

    // ---- per-lane copy plan: LDS slot P of the tile holds global slot (P % spr) ^ swizzle(row);
    //      copy_off[i] is the tile-relative source byte offset of this lane's i-th copy. ----
    std::uint32_t copy_off[kCopies];
#pragma unroll
    for (int i = 0; i < kCopies; ++i) {
        const int p = (wave * kCopies + i) * kWave + lane;
        const int row = p / kSlotsPerRow;
        const int ls = p - row * kSlotsPerRow;
        copy_off[i] = static_cast<std::uint32_t>(row * kDim + (ls ^ swizzle(row)) * 16);
    }
    auto issue = [&](long long item, int slot, int sslot) {
        const long long row0 = phaseBlock(item, phase.stride, phase.skip) * kRows;
        const std::uint8_t* base = corpus + static_cast<std::size_t>(row0) * kDim;
        const std::uint32_t slot_base = ldsAddress(&ring[slot][0]);
        if (row0 + kRows <= doc_count) {
#pragma unroll
            for (int i = 0; i < kCopies; ++i) {
                copyToLds(base, copy_off[i],
                          __builtin_amdgcn_readfirstlane(slot_base + (wave * kCopies + i) * kWave * 16));
            }
        } else {
            // tail tile: rows past the corpus re-read its last row (their scales are NaN)
            const int last = static_cast<int>(doc_count - row0) - 1;
#pragma unroll
            for (int i = 0; i < kCopies; ++i) {
                const int row = static_cast<int>(copy_off[i]) / kDim;
                const std::uint32_t off = copy_off[i] - static_cast<std::uint32_t>((row - min(row, last)) * kDim);
                copyToLds(base, off, __builtin_amdgcn_readfirstlane(slot_base + (wave * kCopies + i) * kWave * 16));
            }
        }
        if (wave == 0 && lane < kRows / 4) {
            // a full tile's 64 scales, or the padded copy of the partial last tile's
            const float* scales = scan.tail_scales != nullptr && row0 + kRows > doc_count ? scan.tail_scales
                                                                                          : scan.row_scales + row0;
            copyToLds(scales, static_cast<std::uint32_t>(16 * lane),
                      __builtin_amdgcn_readfirstlane(ldsAddress(&scale_ring[sslot][0])));
        }
    };

    // prologue: fill the ring up to depth - 1 tiles
    const long long stride_items = gridDim.x;
    long long item = blockIdx.x;
#pragma unroll
    for (int d = 0; d < kDepth - 1; ++d) {
        const long long ahead = item + d * stride_items;
        if (ahead < phase.items) {
            issue(ahead, d, d);
        }
    }
    __syncthreads();  // lds_simd initialization visible

    // Waits for this wavefront's copies of tile `item` (the ones issued after it belong to the at
    // most kDepth - 2 later tiles already in flight) and meets the other wavefronts.
    auto arrive = [&](long long it) {
        int later = 0;
#pragma unroll
        for (int d = 1; d <= kDepth - 2; ++d) {
            later += it + d * stride_items < phase.items ? 1 : 0;
        }
        if (wave == 0) {
            waitTiles<kCopies + 1, kDepth - 2>(later);
        } else {
            waitTiles<kCopies, kDepth - 2>(later);
        }
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");  // no LDS access moves above the barrier
    };
    // Refills the ring slot every wavefront finished reading before the barrier.
    auto refill = [&](long long it, int slot, int sslot) {
        const long long ahead = it + (kDepth - 1) * stride_items;
        if (ahead < phase.items) {
            issue(ahead, slot == 0 ? kDepth - 1 : slot - 1,
                  sslot + kDepth - 1 >= kScaleDepth ? sslot + kDepth - 1 - kScaleDepth : sslot + kDepth - 1);
        }
    };

    // A-fragment addresses. Slot 2 ks + half of row col sits at slot (2 ks + half) ^ swizzle(col)
    // = kSwzSlots (ks / kPeriod) + ((2 (ks % kPeriod) + half) ^ swizzle(col)) with kPeriod =
    // kSwzSlots / 2 k-steps: kPeriod lane-dependent byte offsets; the rest is an immediate (and 32
    // dim bytes for rows 32..63, whose swizzle equals that of rows 0..31).
    constexpr int kPeriod = kSwzSlots / 2;
    std::uint32_t a_off[kPeriod];
#pragma unroll
    for (int m = 0; m < kPeriod; ++m) {
        a_off[m] = static_cast<std::uint32_t>(col * kDim + 16 * ((2 * m + half) ^ swizzle(col)));
    }
    // acc0 = rows 0..31 of the tile x the wavefront's 32 queries, acc1 = rows 32..63. The A
    // fragments run kAhead k-steps ahead of the MFMAs that use them, and the schedule is pinned
    // (reads, then per k-step two MFMAs and the reads kAhead steps further on) so an MFMA never
    // waits on an LDS read issued just before it.
    constexpr int kAhead = kKSteps < 3 ? kKSteps : 3;
    auto multiply = [&](const std::uint8_t* tile, v16i& acc0, v16i& acc1) {
        const std::uint8_t* lane_tile[kPeriod];
#pragma unroll
        for (int m = 0; m < kPeriod; ++m) {
            lane_tile[m] = tile + a_off[m];
        }
        auto fragment = [&](int ks, int half_rows) {
            return *reinterpret_cast<const v4i*>(lane_tile[ks % kPeriod] + 16 * kSwzSlots * (ks / kPeriod) +
                                                 half_rows * 32 * kDim);
        };
        acc0 = v16i{};
        acc1 = v16i{};
        v4i a[kAhead + 1][2];
#pragma unroll
        for (int ks = 0; ks < kAhead; ++ks) {
            a[ks][0] = fragment(ks, 0);
            a[ks][1] = fragment(ks, 1);
        }
#pragma unroll
        for (int ks = 0; ks < kKSteps; ++ks) {
            if (ks + kAhead < kKSteps) {
                a[(ks + kAhead) % (kAhead + 1)][0] = fragment(ks + kAhead, 0);
                a[(ks + kAhead) % (kAhead + 1)][1] = fragment(ks + kAhead, 1);
            }
            acc0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[ks % (kAhead + 1)][0], qf[ks], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[ks % (kAhead + 1)][1], qf[ks], acc1, 0, 0, 0);
        }
        // pinned order: 2 * kAhead LDS reads, then per k-step 2 MFMAs (+ 2 reads while any remain)
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * kAhead, 0);
#pragma unroll
        for (int ks = 0; ks < kKSteps; ++ks) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            if (ks + kAhead < kKSteps) {
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
            }
        }
    };

    int slot = 0;
    int sslot = 0;
    if constexpr (kDense) {
        for (; item < phase.items; item += stride_items) {
            arrive(item);
            refill(item, slot, sslot);
            if (wave_active) {
                v16i acc0;
                v16i acc1;
                multiply(ring[slot], acc0, acc1);
                const long long row0 = phaseBlock(item, phase.stride, phase.skip) * kRows;
                const float* scales = scale_ring[sslot];
                if (q_valid) {
                    std::uint64_t* dst = kStore ? nullptr : emit.dense + static_cast<std::size_t>(q) * emit.dense_stride + item * kRows;
                    float* store = kStore ? emit.scores + static_cast<std::size_t>(q) * doc_count + row0 : nullptr;
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
                                if constexpr (kStore) {
                                    if (row < doc_count) {
                                        store[rl0 + j] = score;
                                    }
                                } else {
                                    dst[rl0 + j] = row < doc_count ? makeKey(score, static_cast<std::uint32_t>(row)) : 0ull;
                                }
                            }
                        }
                    }
                }
            }
            slot = slot + 1 == kDepth ? 0 : slot + 1;
            sslot = sslot + 1 == kScaleDepth ? 0 : sslot + 1;
        }
    } else {
        // leader election: the first wavefront to arrive on each SIMD leads
        bool lead = true;
        {
            std::uint32_t rank = 0u;
            if (lane == 0) {
                rank = atomicAdd(&lds_simd[simdId()], 1u);
            }
            lead = __builtin_amdgcn_readfirstlane(rank) == 0u;
        }

        // relaxed per-lane threshold of the filter; lanes past the launch's queries never pass
        float relaxed_floor = INFINITY;
        if (q_valid) {
            const float t = tau_floor / qscale;
            relaxed_floor = t - fabsf(t) * kFilterMargin - 1e-30f;
        }
        const bool examine_all = __any(q_valid && kMaskedScore >= tau_floor);
        float sketch_best = -INFINITY;  // sketch phases: the lane's best exact score
        // Filter: the wave-uniform set of row groups (group g holds the value slots 4g..4g+3 of
        // a lane: row block g / 4, rows 32 (g / 4) + 8 (g % 4) + 4 half + 0..3, whose scales are
        // one float4) in which some lane's relaxed score (float)dot * s_r reaches the lane's
        // relaxed threshold (tau_floor / s_q, lowered by 2^-20 relative: far more than the
        // few-ulp gap between this product order and the exact score's, so every exact
        // candidate's group is set). A masked or padding row (NaN scale) never passes here; such
        // rows can qualify only against a -FLT_MAX threshold, and then every group is examined.
        auto filter = [&](const v16i& acc0, const v16i& acc1, const float* scales) -> std::uint32_t {
            float4 gs[8];
#pragma unroll
            for (int grp = 0; grp < 8; ++grp) {
                gs[grp] = *reinterpret_cast<const float4*>(scales + (grp / 4) * 32 + 8 * (grp % 4) + 4 * half);
            }
            if constexpr (kSketch) {
                // the sketch: the best exact score of the lane's 32 rows (masked and padding
                // rows score -FLT_MAX), nothing is emitted
#pragma unroll
                for (int grp = 0; grp < 8; ++grp) {
                    const float rsv[4] = {gs[grp].x, gs[grp].y, gs[grp].z, gs[grp].w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int slot = 4 * grp + j;
                        const int dot = slot < 16 ? acc0[slot] : acc1[slot - 16];
                        const float combined = qscale * rsv[j];
                        const float score = rsv[j] == rsv[j] ? static_cast<float>(dot) * combined : kMaskedScore;
                        sketch_best = fmaxf(sketch_best, score);
                    }
                }
                return 0u;
            }
            if (examine_all) {
                return 0xFFu;
            }
            float group_best[8];
#pragma unroll
            for (int grp = 0; grp < 8; ++grp) {
                const float rsv[4] = {gs[grp].x, gs[grp].y, gs[grp].z, gs[grp].w};
                float p[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int slot = 4 * grp + j;
                    const int dot = slot < 16 ? acc0[slot] : acc1[slot - 16];
                    p[j] = static_cast<float>(dot) * rsv[j];
                }
                group_best[grp] = fmaxf(fmaxf(p[0], p[1]), fmaxf(p[2], p[3]));
            }
            const float best = fmaxf(fmaxf(fmaxf(group_best[0], group_best[1]), fmaxf(group_best[2], group_best[3])),
                                     fmaxf(fmaxf(group_best[4], group_best[5]), fmaxf(group_best[6], group_best[7])));
            if (!__any(best >= relaxed_floor)) {
                return 0u;
            }
            std::uint32_t groups = 0u;
#pragma unroll
            for (int grp = 0; grp < 8; ++grp) {
                groups |= (__builtin_amdgcn_ballot_w64(group_best[grp] >= relaxed_floor) != 0ull ? 1u : 0u) << grp;
            }
            return groups;
        };
        const std::uint32_t seg_capacity = 1u << seg_log2;
        // this lane's segment row: segment 2 * workgroup + half, entry `entry`
        const std::size_t seg_row = (static_cast<std::size_t>(2 * blockIdx.x + half) * seg_batch + entry) << seg_log2;
        std::uint32_t seg_used = 0u;  // this lane's candidates so far (may exceed the capacity)
        std::uint32_t parked = 0u;    // wave-uniform: entries of this wavefront's staging buffer
        const std::uint32_t tag = (static_cast<std::uint32_t>(half) << 8) | static_cast<std::uint32_t>(entry - q_offset);
        // Appends `key` for the lanes with `take` set (called by the whole wavefront).
        auto stageCandidates = [&](bool take, std::uint64_t key) {
            const std::uint32_t slot = seg_used;
            seg_used += take ? 1u : 0u;
            const bool store = take && slot < seg_capacity;  // beyond it only counted: overflow
            const std::uint64_t mask = __builtin_amdgcn_ballot_w64(store);
            if (mask == 0ull) {
                return;
            }
            const std::uint32_t rank = __builtin_amdgcn_mbcnt_hi(static_cast<std::uint32_t>(mask >> 32),
                                                                 __builtin_amdgcn_mbcnt_lo(static_cast<std::uint32_t>(mask), 0u));
            const std::uint32_t at = parked + rank;
            parked += static_cast<std::uint32_t>(__builtin_popcountll(mask));
            if (store) {
                if (at < static_cast<std::uint32_t>(kStaged)) {
                    stage_key[wave][at] = key;
                    stage_slot[wave][at] = (slot << 9) | tag;
                } else {
                    emit.seg[seg_row + slot] = key;
                }
            }
        };
        // Exact scores and keys of the row groups `groups` marks; keys above the threshold are
        // appended. One compact loop over the set groups (the group index is wave-uniform, so
        // its accumulator values are picked by register-relative moves; the pass is rare, and the
        // loop keeps the kernel at a third of the code that every group and slot spelled out
        // took, at the same speed). The group's four row scales come in one LDS read from the
        // scale ring, which still holds them, so no scales stay in registers across the barrier.
        auto exact = [&](const v16i& acc0, const v16i& acc1, const float* scales, long long row0,
                         std::uint32_t groups) {
            // Tile-relative rows in 32 bits; the empty asm keeps the compiler from hoisting the
            // per-row constants out of the scan loop into registers.
            int hb = 4 * half;
            asm volatile("" : "+v"(hb));
            const int valid_rows = static_cast<int>(min(static_cast<long long>(kRows), doc_count - row0));
            const std::uint32_t row_base = static_cast<std::uint32_t>(row0);
            while (groups != 0u) {
                const int grp = __builtin_ctz(groups);
                groups &= groups - 1u;
                const int rl0 = (grp >> 2) * 32 + 8 * (grp & 3) + hb;
                const float4 rs4 = *reinterpret_cast<const float4*>(scales + rl0);
                const float rsv[4] = {rs4.x, rs4.y, rs4.z, rs4.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int slot = 4 * grp + j;
                    const int dot = slot < 16 ? acc0[slot] : acc1[slot - 16];
                    const float rs = rsv[j];
                    const float combined = qscale * rs;
                    const float score = rs == rs ? static_cast<float>(dot) * combined : kMaskedScore;
                    const std::uint64_t key = makeKey(score, row_base + static_cast<std::uint32_t>(rl0 + j));
                    stageCandidates(q_valid && rl0 + j < valid_rows && score >= tau_floor && key > tau, key);
                }
            }
        };

        v16i acc0 = {};
        v16i acc1 = {};
        long long acc_row0 = -1;  // first row of the tile in (acc0, acc1); -1 = none yet
        int acc_sslot = 0;
        if (lead) {
            // Leader: multiply tile t, then issue the refill (while the lagger's multiply keeps
            // the matrix core busy) and filter tile t; the exact pass it owes runs after the next
            // barrier, before that step's multiply. (Refilling before the multiply, as the lagger
            // does, measured 1-3% slower per step.)
            std::uint32_t owed = 0u;
            for (; item < phase.items; item += stride_items) {
                arrive(item);
                if (owed != 0u) {
                    exact(acc0, acc1, scale_ring[acc_sslot], acc_row0, owed);
                }
                owed = 0u;
                if (wave_active) {
                    multiply(ring[slot], acc0, acc1);
                    refill(item, slot, sslot);
                    acc_row0 = phaseBlock(item, phase.stride, phase.skip) * kRows;
                    acc_sslot = sslot;
                    owed = filter(acc0, acc1, scale_ring[sslot]);
                } else {
                    refill(item, slot, sslot);
                }
                slot = slot + 1 == kDepth ? 0 : slot + 1;
                sslot = sslot + 1 == kScaleDepth ? 0 : sslot + 1;
            }
            if (owed != 0u) {
                exact(acc0, acc1, scale_ring[acc_sslot], acc_row0, owed);
            }
        } else {
            // Lagger: filter tile t - 1 and run its exact pass, then refill and multiply tile t.
            // (Issuing the refill before the pending exact pass measured slower: the pass's direct
            // stores then queue behind the copies in the vmcnt order.)
            for (; item < phase.items; item += stride_items) {
                arrive(item);
                if (wave_active && acc_row0 >= 0) {
                    const std::uint32_t owed = filter(acc0, acc1, scale_ring[acc_sslot]);
                    if (owed != 0u) {
                        exact(acc0, acc1, scale_ring[acc_sslot], acc_row0, owed);
                    }
                }
                refill(item, slot, sslot);
                if (wave_active) {
                    multiply(ring[slot], acc0, acc1);
                    acc_row0 = phaseBlock(item, phase.stride, phase.skip) * kRows;
                    acc_sslot = sslot;
                }
                slot = slot + 1 == kDepth ? 0 : slot + 1;
                sslot = sslot + 1 == kScaleDepth ? 0 : sslot + 1;
            }
            // the last tile
            if (wave_active && acc_row0 >= 0) {
                const std::uint32_t owed = filter(acc0, acc1, scale_ring[acc_sslot]);
                if (owed != 0u) {
                    exact(acc0, acc1, scale_ring[acc_sslot], acc_row0, owed);
                }
            }
        }

        if constexpr (kSketch) {
            if (q_valid) {
                emit.sketch[static_cast<std::size_t>(2 * blockIdx.x + half) * batch + q] = sketch_best;
            }
            return;
        }
        // write the parked candidates of this wavefront, then every lane's count
        {
            const std::uint32_t held = min(parked, static_cast<std::uint32_t>(kStaged));
            for (std::uint32_t i = static_cast<std::uint32_t>(lane); i < held; i += kWave) {
                const std::uint32_t packed = stage_slot[wave][i];
                const std::size_t segment = 2 * static_cast<std::size_t>(blockIdx.x) + ((packed >> 8) & 1u);
                const std::size_t eg = static_cast<std::size_t>(q_offset) + (packed & 0xFFu);
                emit.seg[((segment * seg_batch + eg) << seg_log2) + (packed >> 9)] = stage_key[wave][i];
            }
        }
        if (q_valid) {
            emit.seg_count[static_cast<std::size_t>(2 * blockIdx.x + half) * seg_batch + entry] = seg_used;
        }
    }
}

template <int kKSteps>
int launchShape(const ScanArgs& scan, const PhaseArgs& phase, const EmitArgs& emit,
                int workgroups, hipStream_t stream) {
    // (a sketch phase fills every workgroup's slots; it gets at least one item per workgroup)
    const long long wanted = phase.dense ? std::min<long long>(phase.items, workgroups) : workgroups;
    const dim3 grid(static_cast<unsigned>(std::max(1LL, wanted)));
    for (int q0 = 0; q0 < scan.batch; q0 += kQueriesPerLaunch) {
        const int count = std::min(kQueriesPerLaunch, scan.batch - q0);
        if (phase.store) {
            mfmaScanKernel<kKSteps, kStoreMode><<<grid, kThreads, 0, stream>>>(scan, phase, emit, q0, count);
        } else if (phase.dense) {
            mfmaScanKernel<kKSteps, kDenseMode><<<grid, kThreads, 0, stream>>>(scan, phase, emit, q0, count);
        } else if (phase.sketch) {
            mfmaScanKernel<kKSteps, kSketchMode><<<grid, kThreads, 0, stream>>>(scan, phase, emit, q0, count);
        } else if (emit.q_list != nullptr) {
            mfmaScanKernel<kKSteps, kRerunMode><<<grid, kThreads, 0, stream>>>(scan, phase, emit, q0, count);
        } else {
            mfmaScanKernel<kKSteps, kThreshold><<<grid, kThreads, 0, stream>>>(scan, phase, emit, q0, count);
        }
        ZCGVS_LAUNCH_CHECK("mfma scan");
    }
    return ZCGVS_OK;
}

}  // namespace

bool mfmaSupported(const ScanArgs& scan) {
    // Below 8 queries the VALU scan (sdot4) is bound by HBM alone, while this kernel would keep
    // seven of its eight wavefronts idle.
    if (scan.batch < kMinBatch) {
        return false;
    }
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

int mfmaSegmentsPerWorkgroup() { return 2; }

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
