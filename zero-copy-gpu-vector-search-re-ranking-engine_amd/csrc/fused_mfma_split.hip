// Float32 rows on the bf16 matrix cores (batches of 32 or more queries, d = 256 or 384): the
// float MFMA scan's contract (fused_mfma_float.hip: scores, keys, segments, dense phase) with the
// products taken as three-part bf16 splits instead of v_mfma_f32_16x16x4_f32, whose rate bounds a
// float32 batch of 64 queries at about twice the time its rows take to stream.
//
// Arithmetic. Every float32 value v (row and query) is split exactly into three bf16 parts by
// truncation: v_h = v with its low 16 bits cleared (sign, exponent, the top 8 significant bits),
// v_m = the same of v - v_h, v_l = v - v_h - v_m (at most 8 significant bits remain, so v_l is a
// bf16 exactly; only values below about 2^-110 lose bits to underflow). The dot product
// sum_j x_j q_j is accumulated in float32 by v_mfma_f32_16x16x32_bf16 as the six part products
// whose weight is at least 2^-16 of the leading one: hh + hm + mh + hl + lh + mm. The three
// dropped products (ml, lm, ll) are below 2^-21 |x_j q_j| together, so a score differs from the
// float32 dot by at most about 2^-21 sum_j |q_j x_j| plus float32 summation rounding.
//
// Work split. A workgroup is 8 wavefronts (two per SIMD) and serves up to 128 queries per
// launch as groups of 16, as in the float MFMA scan: wavefront w keeps the three bf16 parts of
// its group's queries in registers (3 * d / 8 registers per lane) and takes the tile's 16-row
// blocks w / G, w / G + 8 / G, ... (G groups).
//
// Streaming and splitting. A tile is 32 rows. Each lane loads its share of the next tile's
// float32 rows (16-byte chunks, contiguous per wavefront) straight into registers one tile
// ahead, so the loads are in flight while the current tile is multiplied. At the top of a step
// the lane splits its chunks and writes the three parts to a double-buffered LDS plane set
// (each row value is split once per workgroup, not once per query group), the wavefronts meet at
// an LDS-only barrier (the register loads of the next tile stay in flight), and every wavefront
// reads its A fragments from the planes. The query parts take 144 of a wavefront's 256
// registers at d = 384, so one tile (48 KB per workgroup) is all the registers hold in flight. A
// tile takes about 2.9 us against 1.3 us of MFMA work; its LDS traffic (288 KB of A fragments
// read and 72 KB of planes written per 48 KB tile) is of the same order as the matrix core's
// time, and a form with two tiles in flight (pairs of wavefronts splitting the dimensions,
// single-buffered planes) was slower. Plane row r keeps its 16-byte chunk s (8 dims) at chunk
// s ^ (r & 15) (rows are whole multiples of 256 bytes), so the 16 rows one ds_read_b128 quarter-
// wave reads hit 16 distinct bank groups.
//
// MFMA layout (16x16x32 bf16, wave64): A (16 rows x 32 dims): lane l supplies row l % 16 and the
// 8 dims 8 (l / 16) .. + 7 of the step; B (32 dims x 16 queries): lane l supplies query l % 16
// with the same dims. D: lane l holds query l % 16 and rows 4 (l / 16) + i, i < 4.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.hpp"
#include "fused.hpp"
#include "lds_copy.hpp"
#include "scan_core.hpp"

namespace zcgvs_hip {

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int kGroupQueries = 16;
constexpr int kQueriesPerLaunch = kWaves * kGroupQueries;
constexpr int kRows = 32;        // tile rows: two 16-row blocks
constexpr int kMinQueries = 32;  // launches with fewer queries keep the float32 MFMA scan

template <int kDim>
struct SplitTile {
    static constexpr int kChunks = kDim / 4;                   // 16-byte float32 chunks per row
    static constexpr int kLoads = kRows * kChunks / kThreads;  // chunks per lane per tile
    static constexpr int kPlaneRow = kDim * 2;                 // bytes of one row of one part
    static constexpr int kPlaneBytes = kRows * kPlaneRow;
    static constexpr int kSteps = kDim / 32;
    static_assert(kRows * kChunks % kThreads == 0, "a tile splits evenly over the lanes");
    static_assert(kPlaneRow % 256 == 0, "plane rows are whole multiples of 256 bytes");
    static_assert(2 * 3 * kPlaneBytes + 4 * kQueriesPerLaunch <= 160 * 1024, "planes fit the LDS");
};

// The three bf16 parts of four float32 values, packed two per word (low half = lower dim).
struct Parts4 {
    unsigned h[2], m[2], l[2];
};

__device__ __forceinline__ Parts4 splitFour(v4u bits) {
    Parts4 p;
    unsigned hb[4], mb[4], lb[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float v = __uint_as_float(bits[e]);
        hb[e] = bits[e] & 0xFFFF0000u;
        const float r1 = v - __uint_as_float(hb[e]);
        mb[e] = __float_as_uint(r1) & 0xFFFF0000u;
        const float r2 = r1 - __uint_as_float(mb[e]);
        lb[e] = __float_as_uint(r2);  // its low 16 bits are zero
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        p.h[k] = (hb[2 * k] >> 16) | hb[2 * k + 1];
        p.m[k] = (mb[2 * k] >> 16) | mb[2 * k + 1];
        p.l[k] = (lb[2 * k] >> 16) | (lb[2 * k + 1] & 0xFFFF0000u);
    }
    return p;
}

__device__ __forceinline__ void ldsBarrierSplit() {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wavefront's LDS writes are done
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int kDim, bool kDense>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void mfmaSplitScanKernel(ScanArgs scan, PhaseArgs phase, EmitArgs emit, int q_offset, int q_count) {
    using Tile = SplitTile<kDim>;
    constexpr int kChunks = Tile::kChunks;
    constexpr int kLoads = Tile::kLoads;
    constexpr int kPlaneRow = Tile::kPlaneRow;
    constexpr int kPlaneBytes = Tile::kPlaneBytes;
    constexpr int kSteps = Tile::kSteps;
    constexpr int kRowBlocks = kRows / 16;

    __shared__ __attribute__((aligned(16))) std::uint8_t planes[2][3][kPlaneBytes];
    __shared__ std::uint32_t lds_count[kQueriesPerLaunch];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int r16 = lane & 15;
    const int h = lane >> 4;
    const int groups = (q_count + kGroupQueries - 1) / kGroupQueries;
    const int waves_per_group = kWaves / groups;
    const bool wave_active = wave < groups * waves_per_group;
    const int group = wave % groups;
    const int first_block = wave / groups;
    const int qlocal = group * kGroupQueries + r16;
    const bool q_valid = wave_active && qlocal < q_count;
    const int q = q_offset + min(qlocal, q_count - 1);
    const long long doc_count = scan.doc_count;
    const std::uint8_t* corpus = static_cast<const std::uint8_t*>(scan.corpus);

    // ---- query parts: step t holds dims 32 t + 8 h .. + 7 ----
    v8bf qh[kSteps], qm[kSteps], ql[kSteps];
    {
        const float* qrow = static_cast<const float*>(scan.queries) + static_cast<std::size_t>(q) * kDim;
#pragma unroll
        for (int t = 0; t < kSteps; ++t) {
            v4u words_h, words_m, words_l;
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                v4u bits = *reinterpret_cast<const v4u*>(qrow + 32 * t + 8 * h + 4 * p);
                if (!q_valid) {
                    bits = v4u{0u, 0u, 0u, 0u};
                }
                const Parts4 s = splitFour(bits);
                words_h[2 * p] = s.h[0];
                words_h[2 * p + 1] = s.h[1];
                words_m[2 * p] = s.m[0];
                words_m[2 * p + 1] = s.m[1];
                words_l[2 * p] = s.l[0];
                words_l[2 * p + 1] = s.l[1];
            }
            qh[t] = __builtin_bit_cast(v8bf, words_h);
            qm[t] = __builtin_bit_cast(v8bf, words_m);
            ql[t] = __builtin_bit_cast(v8bf, words_l);
        }
    }
    std::uint64_t tau = 0ull;
    if constexpr (!kDense) {
        tau = emit.tau[q];
    }
    for (int i = tid; i < kQueriesPerLaunch; i += kThreads) {
        lds_count[i] = 0u;
    }

    // ---- this lane's chunks of a tile: chunk p = (wave * kLoads + i) * 64 + lane of the tile's
    //      rows * kChunks chunks, i.e. row p / kChunks, chunk p % kChunks (recomputed at each use:
    //      registers are short) ----
    auto chunkOf = [&](int i, int& row, int& c) __attribute__((always_inline)) {
        const int p = (wave * kLoads + i) * kWave + lane;
        row = p / kChunks;
        c = p - row * kChunks;
    };
    v4u raw[kLoads];
    auto load = [&](long long it) __attribute__((always_inline)) {
        const long long row0 = phaseBlock(it, phase.stride, phase.skip) * kRows;
        const std::uint8_t* base = corpus + static_cast<std::size_t>(row0) * kDim * 4;
        const int last = static_cast<int>(min(static_cast<long long>(kRows), doc_count - row0)) - 1;
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            int row, c;
            chunkOf(i, row, c);
            // rows past the corpus re-read its last row (never emitted)
            const std::uint32_t off = static_cast<std::uint32_t>(min(row, last) * kDim * 4 + c * 16);
            raw[i] = __builtin_bit_cast(v4u, loadChunkStreaming(base + off));
        }
    };
    auto store = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            int row, c;
            chunkOf(i, row, c);
            // its 8 bytes: half c % 2 of plane chunk c / 2, swizzled within the row
            const int dst = row * kPlaneRow + (((c >> 1) ^ (row & 15)) * 16) + (c & 1) * 8;
            const Parts4 s = splitFour(raw[i]);
            *reinterpret_cast<uint2*>(&planes[buf][0][dst]) = make_uint2(s.h[0], s.h[1]);
            *reinterpret_cast<uint2*>(&planes[buf][1][dst]) = make_uint2(s.m[0], s.m[1]);
            *reinterpret_cast<uint2*>(&planes[buf][2][dst]) = make_uint2(s.l[0], s.l[1]);
        }
    };

    // A fragment of step t for row r16 of a block: chunk 4 t + h of the row, swizzled.
    std::uint32_t a_off[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        a_off[m] = static_cast<std::uint32_t>(r16 * kPlaneRow + ((4 * m + h) ^ r16) * 16);
    }
    // Scores of 16-row block `block` of plane set `buf` for this lane's query (rows 4 h + i).
    // The A fragments of the three parts run kAhead steps ahead of their MFMAs.
    constexpr int kAhead = kSteps < 2 ? kSteps : 2;
    auto multiply = [&](int buf, int block) __attribute__((always_inline)) -> v4f {
        const std::uint8_t* rows_h = &planes[buf][0][block * 16 * kPlaneRow];
        const std::uint8_t* rows_m = &planes[buf][1][block * 16 * kPlaneRow];
        const std::uint8_t* rows_l = &planes[buf][2][block * 16 * kPlaneRow];
        auto fragment = [&](const std::uint8_t* rows, int t) {
            return *reinterpret_cast<const v8bf*>(rows + a_off[t % 4] + 256 * (t / 4));
        };
        v4f acc0 = {0.0f, 0.0f, 0.0f, 0.0f};
        v4f acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
        v8bf ah[kAhead + 1], am[kAhead + 1], al[kAhead + 1];
#pragma unroll
        for (int t = 0; t < kAhead; ++t) {
            ah[t] = fragment(rows_h, t);
            am[t] = fragment(rows_m, t);
            al[t] = fragment(rows_l, t);
        }
#pragma unroll
        for (int t = 0; t < kSteps; ++t) {
            if (t + kAhead < kSteps) {
                const int n = (t + kAhead) % (kAhead + 1);
                ah[n] = fragment(rows_h, t + kAhead);
                am[n] = fragment(rows_m, t + kAhead);
                al[n] = fragment(rows_l, t + kAhead);
            }
            const int c = t % (kAhead + 1);
            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[c], qh[t], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[c], qm[t], acc1, 0, 0, 0);
            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am[c], qh[t], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[c], ql[t], acc1, 0, 0, 0);
            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am[c], qm[t], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[c], qh[t], acc1, 0, 0, 0);
        }
        // pinned order: the first reads, then per step its six MFMAs and the reads kAhead on
        __builtin_amdgcn_sched_group_barrier(0x100, 3 * kAhead, 0);
#pragma unroll
        for (int t = 0; t < kSteps; ++t) {
            __builtin_amdgcn_sched_group_barrier(0x008, 6, 0);
            if (t + kAhead < kSteps) {
                __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
            }
        }
        return acc0 + acc1;
    };

    // Per tile: wait for this lane's chunks, split them into the free plane set, start the next
    // tile's loads (they stay in flight through the barrier and the multiply), meet at an
    // LDS-only barrier, multiply. (Splitting the next tile inside the current multiply instead,
    // to overlap the split with the matrix core, measured 3% slower.)
    const long long stride_items = gridDim.x;
    long long item = blockIdx.x;
    if (item < phase.items) {
        load(item);
    }
    __syncthreads();  // lds_count initialization visible
    int buf = 0;
    for (; item < phase.items; item += stride_items) {
        __builtin_amdgcn_s_waitcnt(vmcntOnly(0));  // this lane's chunks of tile `item`
        store(buf);
        if (item + stride_items < phase.items) {
            load(item + stride_items);
        }
        ldsBarrierSplit();
        if (wave_active) {
            const long long row0 = phaseBlock(item, phase.stride, phase.skip) * kRows;
            for (int block = first_block; block < kRowBlocks; block += waves_per_group) {
                const v4f score = multiply(buf, block);
                if (q_valid) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int local = block * 16 + 4 * h + i;
                        const long long row = row0 + local;
                        const std::uint64_t key =
                            row < doc_count ? makeKey(score[i], static_cast<std::uint32_t>(row)) : 0ull;
                        if constexpr (kDense) {
                            emit.dense[static_cast<std::size_t>(q) * emit.dense_stride + item * kRows + local] = key;
                        } else if (key > tau) {
                            appendCandidate(emit, lds_count, q, q_offset, scan.batch, key);
                        }
                    }
                }
            }
        }
        buf ^= 1;
    }
    if constexpr (!kDense) {
        __syncthreads();
        for (int i = tid; i < q_count; i += kThreads) {
            emit.seg_count[static_cast<std::size_t>(blockIdx.x) * scan.batch + q_offset + i] = lds_count[i];
        }
    }
}

template <int kDim>
int launchSplitDim(const ScanArgs& scan, const PhaseArgs& phase, const EmitArgs& emit, dim3 grid, int q0,
                   int count, hipStream_t stream) {
    if (phase.dense) {
        mfmaSplitScanKernel<kDim, true><<<grid, kThreads, 0, stream>>>(scan, phase, emit, q0, count);
    } else {
        mfmaSplitScanKernel<kDim, false><<<grid, kThreads, 0, stream>>>(scan, phase, emit, q0, count);
    }
    ZCGVS_LAUNCH_CHECK("split mfma scan");
    return ZCGVS_OK;
}

}  // namespace

int mfmaSplitRows() { return kRows; }

bool mfmaSplitSupported(const ScanArgs& scan, int queries_in_launch) {
    return scan.dtype == ZCGVS_DTYPE_F32 && scan.lexical == nullptr && scan.mask == nullptr &&
           (scan.dim == 256 || scan.dim == 384) && queries_in_launch >= kMinQueries &&
           queries_in_launch <= kQueriesPerLaunch &&
           (scan.metric == ZCGVS_METRIC_COSINE || scan.metric == ZCGVS_METRIC_DOT) && aligned16(scan.corpus) &&
           aligned16(scan.queries);
}

int launchMfmaSplitScan(const ScanArgs& scan, const PhaseArgs& phase, const EmitArgs& emit, int workgroups,
                        int q0, int count, hipStream_t stream) {
    if (!mfmaSplitSupported(scan, count)) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: split MFMA scan does not take this shape");
    }
    const long long wanted = phase.dense ? std::min<long long>(phase.items, workgroups) : workgroups;
    const dim3 grid(static_cast<unsigned>(std::max(1LL, wanted)));
    return scan.dim == 256 ? launchSplitDim<256>(scan, phase, emit, grid, q0, count, stream)
                           : launchSplitDim<384>(scan, phase, emit, grid, q0, count, stream);
}

}  // namespace zcgvs_hip
