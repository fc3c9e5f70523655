// Float MFMA fused scan: float32 or float16 corpus rows against a batch of float32 queries, on
// the matrix cores, with the threshold emission of fused.hpp in the epilogue. It replaces the
// reference's per-lane FMA loop (src/cuda/similarity.cu:83-164 with accumulateMetric of
// include/zcgvs/cuda/decode.cuh:30-42: dot and cosine both accumulate q * x) for batches, where
// that loop re-streams the corpus once per 8 queries and is bound by its query reads.
//
// Arithmetic.
//   float32 rows: v_mfma_f32_16x16x4_f32, float32 products and sums, i.e. the same operation as
//   the scalar loop in another summation order (scores agree to float32 rounding).
//   float16 rows: v_mfma_f32_16x16x32_f16. The stored halves enter exactly; each query is split
//   into two halves q * 2^e = hi + lo (hi = half(q * 2^e), lo = half(q * 2^e - hi), with 2^e the
//   power of two that brings the query's largest |q_j| to [2^14, 2^15)), both products are
//   accumulated in float32 and the sum is scaled back by 2^-e. The split keeps 22 significant
//   bits of every q_j, so a score differs from the float32 dot of the widened row by at most
//   about 2^-22 * sum_j |q_j x_j| plus float32 summation rounding (components of q below
//   2^-38 * max |q| are lost in the split).
//
// Work split. A workgroup is 8 wavefronts, two per SIMD, and serves up to 128 queries per launch
// as groups of 16. Wavefront w takes query group w % G (G groups in the launch) and keeps that
// group's query values in registers for the whole launch as MFMA B operands (query-stationary):
// kDim / 4 registers per lane for both kinds. With fewer than 8 groups the wavefronts of a group
// split the tile's 16-row blocks between them.
//
// MFMA layout (16x16xK, wave64). A (16 x K, rows x dims): lane l supplies row l % 16 and the K/4
// dims of lane group l / 16; B (K x 16, dims x queries): lane l supplies query l % 16 with the
// same dims, so the product sums every dim exactly once whatever order the hardware uses. One
// ds_read_b128 gives a lane the 16 bytes of chunk 4t + l / 16 of its row: 8 halves (one f16
// MFMA) or 4 floats (four f32 MFMAs, component c of every lane group forming the c-th).
// D: lane l holds query l % 16 and rows 4 * (l / 16) + i, i < 4.
//
// Hybrid searches (lexical scores fused into the dense score, fuseHybrid of fused.hpp) take up
// to 16 queries per launch; each tile's [16, rows] block of lexical scores travels HBM -> LDS
// with global_load_lds_dword in a ring beside the tile ring, so the epilogue reads LDS only (a
// plain global load there would make the compiler wait for every copy in flight).
//
// Corpus streaming is the one of the int8 MFMA scan (lds_copy.hpp): tiles of whole rows go HBM ->
// LDS through global_load_lds_dwordx4 into a ring kDepth - 1 tiles ahead; every wavefront waits
// for its own copies of a tile and meets the others at a bare s_barrier. Tile rows are sized so
// a tile holds about 48 KB. LDS slot s of row r holds the row's 16-byte chunk s ^ (r & 15) (rows
// are whole multiples of 256 bytes), so the 16 rows one ds_read_b128 quarter-wave reads hit 16
// distinct bank groups.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.hpp"
#include "fused.hpp"
#include "lds_copy.hpp"

namespace zcgvs_hip {

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int kGroupQueries = 16;
constexpr int kQueriesPerLaunch = kWaves * kGroupQueries;
constexpr int kTileTarget = 48 * 1024;
constexpr int kRingBudget = 150 * 1024;
constexpr int kMinBatch = 4;  // below this the VALU scan is already bound by HBM
constexpr int kLexQueries = 16;  // queries per launch of a hybrid search

constexpr int pow2Floor(int value) {
    int p = 1;
    while (2 * p <= value) {
        p *= 2;
    }
    return p;
}

template <int kKind, int kDim>
struct FloatTile {
    static constexpr bool kF32 = kKind == ZCGVS_DTYPE_F32;
    static constexpr int kRowBytes = kDim * (kF32 ? 4 : 2);
    static constexpr int kChunks = kRowBytes / 16;
    static constexpr int kSteps = kChunks / 4;  // ds_read_b128 steps per row
    static constexpr int kRowsRaw = pow2Floor(kTileTarget / kRowBytes);
    static constexpr int kRows = kRowsRaw < 16 ? 16 : (kRowsRaw > 128 ? 128 : kRowsRaw);
    static constexpr int kTileBytes = kRows * kRowBytes;
    static constexpr int kDepth = 3 * kTileBytes <= kRingBudget ? 3 : 2;
    static constexpr int kCopies = kRows * kChunks / kThreads;  // 16-byte copies per lane per tile
    static_assert(kRowBytes % 256 == 0, "rows must be whole multiples of 256 bytes");
    static_assert(kRows * kChunks % kThreads == 0, "tile must split over the lanes");
    static_assert(2 * kCopies < 63, "copies in flight fit the vmcnt counter");
    // lexical ring of hybrid launches: [kDepth][kLexQueries][kLexStride] floats; each wave
    // copies the rows of queries w and w + 8, 64 rows per dword copy
    static constexpr int kLexStride = kRows < kWave ? kWave : kRows;
    static constexpr int kLexPieces = (kRows + kWave - 1) / kWave;
    static constexpr int kLexCopies = 2 * kLexPieces;
    static_assert(kDepth * (kTileBytes + kLexQueries * kLexStride * 4) + 4 * kQueriesPerLaunch <= 160 * 1024,
                  "tile and lexical rings fit the LDS");
};

template <int kKind, int kDim, bool kDense, bool kLex, bool kStore = false>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void mfmaFloatScanKernel(ScanArgs scan, PhaseArgs phase, EmitArgs emit, int q_offset, int q_count) {
    static_assert(!kStore || (kDense && !kLex), "a store phase is a dense phase without lexical scores");
    using Tile = FloatTile<kKind, kDim>;
    constexpr bool kF32 = Tile::kF32;
    constexpr int kRows = Tile::kRows;
    constexpr int kRowBytes = Tile::kRowBytes;
    constexpr int kChunks = Tile::kChunks;
    constexpr int kSteps = Tile::kSteps;
    constexpr int kDepth = Tile::kDepth;
    constexpr int kCopies = Tile::kCopies;
    constexpr int kRowBlocks = kRows / 16;
    constexpr int kLexStride = Tile::kLexStride;
    constexpr int kLexPieces = Tile::kLexPieces;
    constexpr int kPerTile = kCopies + (kLex ? Tile::kLexCopies : 0);  // copies per wave per tile

    __shared__ __attribute__((aligned(16))) std::uint8_t ring[kDepth][Tile::kTileBytes];
    __shared__ std::uint32_t lds_count[kQueriesPerLaunch];
    __shared__ float lex_ring[kLex ? kDepth : 1][kLex ? kLexQueries : 1][kLex ? kLexStride : 1];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // wave-uniform: scalar indexing
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

    // ---- query fragments: step t holds dims 16t + 4h .. +3 (f32) or 32t + 8h .. +7 (f16) ----
    const float* qrow = static_cast<const float*>(scan.queries) + static_cast<std::size_t>(q) * kDim;
    v4f qf[kF32 ? kSteps : 1];
    v8h qhi[kF32 ? 1 : kSteps];
    v8h qlo[kF32 ? 1 : kSteps];
    float unscale = 1.0f;
    if constexpr (kF32) {
#pragma unroll
        for (int t = 0; t < kSteps; ++t) {
            const v4f value = *reinterpret_cast<const v4f*>(qrow + 16 * t + 4 * h);
            qf[t] = q_valid ? value : v4f{0.0f, 0.0f, 0.0f, 0.0f};
        }
    } else {
        v4f raw[kSteps][2];
        float peak = 0.0f;
#pragma unroll
        for (int t = 0; t < kSteps; ++t) {
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const v4f value = *reinterpret_cast<const v4f*>(qrow + 32 * t + 8 * h + 4 * p);
                raw[t][p] = q_valid ? value : v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    peak = fmaxf(peak, fabsf(raw[t][p][e]));
                }
            }
        }
        // the four lanes of a query (l, l ^ 16, l ^ 32, l ^ 48) agree on its largest |q_j|
        peak = fmaxf(peak, waveXor(peak, 16));
        peak = fmaxf(peak, waveXor(peak, 32));
        int exponent = 0;
        if (peak > 0.0f && peak <= 3.402823466e+38f) {
            int e = 0;
            frexpf(peak, &e);  // peak = m * 2^e, m in [0.5, 1)
            exponent = min(126, max(-126, 15 - e));
        }
        const float scale = ldexpf(1.0f, exponent);
        unscale = ldexpf(1.0f, -exponent);
#pragma unroll
        for (int t = 0; t < kSteps; ++t) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float x = raw[t][e / 4][e % 4] * scale;
                const _Float16 hi = static_cast<_Float16>(x);
                qhi[t][e] = hi;
                qlo[t][e] = static_cast<_Float16>(x - static_cast<float>(hi));
            }
        }
    }
    std::uint64_t tau = 0ull;
    bool gated = false;  // tau_floor applies (every key above tau scores at least tau_floor)
    float tau_floor = 0.0f;
    if constexpr (!kDense) {
        tau = emit.tau[q];
        tau_floor = keyFloor(tau, &gated);
    }
    float inverse = 0.0f;  // 1 / (the query's largest lexical score), 0 when none is positive
    if constexpr (kLex) {
        const float peak = scan.lexical_max[q];
        inverse = peak > 0.0f ? 1.0f / peak : 0.0f;
    }
    for (int i = tid; i < kQueriesPerLaunch; i += kThreads) {
        lds_count[i] = 0u;
    }

    // ---- copy plan: LDS slot P of a tile holds chunk (P % kChunks) ^ (row & 15) of its row ----
    std::uint32_t copy_off[kCopies];
#pragma unroll
    for (int i = 0; i < kCopies; ++i) {
        const int p = (wave * kCopies + i) * kWave + lane;
        const int row = p / kChunks;
        const int slot = p - row * kChunks;
        copy_off[i] = static_cast<std::uint32_t>(row * kRowBytes + (slot ^ (row & 15)) * 16);
    }
    auto issue = [&](long long item, int slot) {
        const long long row0 = phaseBlock(item, phase.stride, phase.skip) * kRows;
        const std::uint8_t* base = corpus + static_cast<std::size_t>(row0) * kRowBytes;
        const std::uint32_t slot_base = ldsAddress(&ring[slot][0]);
        if (row0 + kRows <= doc_count) {
#pragma unroll
            for (int i = 0; i < kCopies; ++i) {
                copyToLds(base, copy_off[i],
                          __builtin_amdgcn_readfirstlane(slot_base + (wave * kCopies + i) * kWave * 16));
            }
        } else {
            // partial last tile: rows past the corpus re-read its last row (and are never emitted)
            const int last = static_cast<int>(doc_count - row0) - 1;
#pragma unroll
            for (int i = 0; i < kCopies; ++i) {
                const int row = static_cast<int>(copy_off[i]) / kRowBytes;
                const std::uint32_t off = copy_off[i] - static_cast<std::uint32_t>((row - min(row, last)) * kRowBytes);
                copyToLds(base, off, __builtin_amdgcn_readfirstlane(slot_base + (wave * kCopies + i) * kWave * 16));
            }
        }
        if constexpr (kLex) {
            // rows row0 + 64 p + lane of queries wave and wave + 8 (rows past the corpus re-read
            // its last row; a missing query re-reads query 0's scores; neither is ever used)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int ql = wave + 8 * j;
                const long long qg = q_offset + (ql < q_count ? ql : 0);
#pragma unroll
                for (int p = 0; p < kLexPieces; ++p) {
                    const long long row = min(row0 + kWave * p + lane, doc_count - 1);
                    copyDwordToLds(scan.lexical + qg * doc_count + row,
                                   __builtin_amdgcn_readfirstlane(ldsAddress(&lex_ring[slot][ql][kWave * p])));
                }
            }
        }
    };

    const long long stride_items = gridDim.x;
    long long item = blockIdx.x;
#pragma unroll
    for (int d = 0; d < kDepth - 1; ++d) {
        if (item + d * stride_items < phase.items) {
            issue(item + d * stride_items, d);
        }
    }
    __syncthreads();  // lds_count initialization visible

    auto arrive = [&](long long it) {
        int later = 0;
#pragma unroll
        for (int d = 1; d <= kDepth - 2; ++d) {
            later += it + d * stride_items < phase.items ? 1 : 0;
        }
        waitTiles<kPerTile, kDepth - 2>(later);
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");  // no LDS access moves above the barrier
    };

    // A-fragment offsets: chunk 4t + h of row r16 sits at 256 * (t / 4) + ((4 (t % 4) + h) ^ r16) * 16.
    std::uint32_t a_off[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        a_off[m] = static_cast<std::uint32_t>(r16 * kRowBytes + ((4 * m + h) ^ r16) * 16);
    }
    // Scores of the 16-row block `block` of a tile for this lane's query: rows 4h + i. Two
    // accumulator chains (f32: even / odd components; f16: hi / lo query halves) are summed at
    // the end. A fragments run kAhead steps ahead of their MFMAs.
    constexpr int kAhead = kSteps < 3 ? kSteps : 3;
    auto multiply = [&](const std::uint8_t* tile, int block) -> v4f {
        const std::uint8_t* rows = tile + block * 16 * kRowBytes;
        auto fragment = [&](int t) {
            return *reinterpret_cast<const v4f*>(rows + a_off[t % 4] + 256 * (t / 4));
        };
        v4f acc0 = {0.0f, 0.0f, 0.0f, 0.0f};
        v4f acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
        v4f a[kAhead + 1];
#pragma unroll
        for (int t = 0; t < kAhead; ++t) {
            a[t] = fragment(t);
        }
#pragma unroll
        for (int t = 0; t < kSteps; ++t) {
            if (t + kAhead < kSteps) {
                a[(t + kAhead) % (kAhead + 1)] = fragment(t + kAhead);
            }
            const v4f frag = a[t % (kAhead + 1)];
            if constexpr (kF32) {
                acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(frag[0], qf[t][0], acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(frag[1], qf[t][1], acc1, 0, 0, 0);
                acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(frag[2], qf[t][2], acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(frag[3], qf[t][3], acc1, 0, 0, 0);
            } else {
                const v8h halves = __builtin_bit_cast(v8h, frag);
                acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(halves, qhi[t], acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(halves, qlo[t], acc1, 0, 0, 0);
            }
        }
        // pinned order: kAhead reads, then per step its MFMAs and the read kAhead steps further on
        constexpr int kMfmaPerStep = kF32 ? 4 : 2;
        __builtin_amdgcn_sched_group_barrier(0x100, kAhead, 0);
#pragma unroll
        for (int t = 0; t < kSteps; ++t) {
            __builtin_amdgcn_sched_group_barrier(0x008, kMfmaPerStep, 0);
            if (t + kAhead < kSteps) {
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
        }
        v4f score;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            score[i] = kF32 ? acc0[i] + acc1[i] : (acc0[i] + acc1[i]) * unscale;
        }
        return score;
    };

    int slot = 0;
    for (; item < phase.items; item += stride_items) {
        arrive(item);
        {
            const long long ahead = item + (kDepth - 1) * stride_items;
            if (ahead < phase.items) {
                issue(ahead, slot == 0 ? kDepth - 1 : slot - 1);
            }
        }
        if (wave_active) {
            const long long row0 = phaseBlock(item, phase.stride, phase.skip) * kRows;
            const int valid_rows = static_cast<int>(min(static_cast<long long>(kRows), doc_count - row0));
            const std::uint32_t row_base = static_cast<std::uint32_t>(row0);
            for (int block = first_block; block < kRowBlocks; block += waves_per_group) {
                const v4f score = multiply(ring[slot], block);
                if (q_valid) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int local = block * 16 + 4 * h + i;
                        float value = score[i];
                        if constexpr (kLex) {
                            value = fuseHybrid(value, lex_ring[slot][qlocal][local], scan.dense_weight, inverse);
                        }
                        if constexpr (kStore) {
                            if (local < valid_rows) {
                                emit.scores[static_cast<std::size_t>(q) * doc_count + row0 + local] = value;
                            }
                        } else if constexpr (kDense) {
                            const std::uint64_t key =
                                local < valid_rows ? makeKey(value, row_base + static_cast<std::uint32_t>(local)) : 0ull;
                            emit.dense[static_cast<std::size_t>(q) * emit.dense_stride + item * kRows + local] = key;
                        } else if (!gated || value >= tau_floor) {
                            // (almost every row of a threshold phase fails the score test above)
                            const std::uint64_t key =
                                local < valid_rows ? makeKey(value, row_base + static_cast<std::uint32_t>(local)) : 0ull;
                            if (key > tau) {
                                appendCandidate(emit, lds_count, q, q_offset, scan.batch, key);
                            }
                        }
                    }
                }
            }
        }
        slot = slot + 1 == kDepth ? 0 : slot + 1;
    }
    if constexpr (!kDense) {
        __syncthreads();
        for (int i = tid; i < q_count; i += kThreads) {
            emit.seg_count[static_cast<std::size_t>(blockIdx.x) * scan.batch + q_offset + i] = lds_count[i];
        }
    }
}

template <int kKind, int kDim, bool kLex>
int launchQueries(const ScanArgs& scan, const PhaseArgs& phase, const EmitArgs& emit, dim3 grid,
                  hipStream_t stream) {
    const int per_launch = kLex ? kLexQueries : kQueriesPerLaunch;
    for (int q0 = 0; q0 < scan.batch; q0 += per_launch) {
        const int count = std::min(per_launch, scan.batch - q0);
        if (kKind == ZCGVS_DTYPE_F32 && !kLex && !phase.store && mfmaSplitSupported(scan, count)) {
            // float32 rows against 32 or more queries: the bf16 three-part split scan, whose
            // 32-row tiles and emission are this kernel's
            static_assert(kKind != ZCGVS_DTYPE_F32 || kDim < 256 || kDim > 384 || FloatTile<kKind, kDim>::kRows == 32,
                          "the split scan uses 32-row tiles");
            const int status = launchMfmaSplitScan(scan, phase, emit, static_cast<int>(grid.x), q0, count, stream);
            if (status != ZCGVS_OK) {
                return status;
            }
            continue;
        }
        if (phase.store) {
            if constexpr (!kLex) {
                mfmaFloatScanKernel<kKind, kDim, true, false, true><<<grid, kThreads, 0, stream>>>(scan, phase, emit, q0,
                                                                                                    count);
            }
        } else if (phase.dense) {
            mfmaFloatScanKernel<kKind, kDim, true, kLex><<<grid, kThreads, 0, stream>>>(scan, phase, emit, q0, count);
        } else {
            mfmaFloatScanKernel<kKind, kDim, false, kLex><<<grid, kThreads, 0, stream>>>(scan, phase, emit, q0, count);
        }
        ZCGVS_LAUNCH_CHECK("float mfma scan");
    }
    return ZCGVS_OK;
}

template <int kKind, int kDim>
int launchShape(const ScanArgs& scan, const PhaseArgs& phase, const EmitArgs& emit, int workgroups,
                hipStream_t stream) {
    const long long wanted = phase.dense ? std::min<long long>(phase.items, workgroups) : workgroups;
    const dim3 grid(static_cast<unsigned>(std::max(1LL, wanted)));
    return scan.lexical != nullptr ? launchQueries<kKind, kDim, true>(scan, phase, emit, grid, stream)
                                   : launchQueries<kKind, kDim, false>(scan, phase, emit, grid, stream);
}

// Calls f(FloatTile<kind, dim>-shaped tag) for the supported (kind, dim) pairs; false otherwise.
template <typename F>
bool dispatchShape(int kind, int dim, F&& f) {
#define ZCGVS_FLOAT_SHAPE(KIND, DIM) \
    if (kind == KIND && dim == DIM) { f.template operator()<KIND, DIM>(); return true; }
    ZCGVS_FLOAT_SHAPE(ZCGVS_DTYPE_F32, 128)
    ZCGVS_FLOAT_SHAPE(ZCGVS_DTYPE_F32, 256)
    ZCGVS_FLOAT_SHAPE(ZCGVS_DTYPE_F32, 384)
    ZCGVS_FLOAT_SHAPE(ZCGVS_DTYPE_F32, 512)
    ZCGVS_FLOAT_SHAPE(ZCGVS_DTYPE_F16, 128)
    ZCGVS_FLOAT_SHAPE(ZCGVS_DTYPE_F16, 256)
    ZCGVS_FLOAT_SHAPE(ZCGVS_DTYPE_F16, 384)
    ZCGVS_FLOAT_SHAPE(ZCGVS_DTYPE_F16, 512)
#undef ZCGVS_FLOAT_SHAPE
    return false;
}

struct RowsOf {
    int rows = 0;
    template <int kKind, int kDim>
    void operator()() { rows = FloatTile<kKind, kDim>::kRows; }
};

struct Launch {
    const ScanArgs& scan;
    const PhaseArgs& phase;
    const EmitArgs& emit;
    int workgroups;
    hipStream_t stream;
    int status = ZCGVS_OK;
    template <int kKind, int kDim>
    void operator()() { status = launchShape<kKind, kDim>(scan, phase, emit, workgroups, stream); }
};

}  // namespace

bool mfmaFloatSupported(const ScanArgs& scan) {
    if (scan.dtype != ZCGVS_DTYPE_F32 && scan.dtype != ZCGVS_DTYPE_F16) {
        return false;
    }
    if (scan.metric != ZCGVS_METRIC_COSINE && scan.metric != ZCGVS_METRIC_DOT) {
        return false;
    }
    if (scan.mask != nullptr || scan.batch < kMinBatch) {
        return false;
    }
    if (!aligned16(scan.corpus) || !aligned16(scan.queries)) {
        return false;
    }
    RowsOf probe;
    return dispatchShape(scan.dtype, scan.dim, probe);
}

int mfmaFloatBlockRows(const ScanArgs& scan) {
    RowsOf probe;
    dispatchShape(scan.dtype, scan.dim, probe);
    return probe.rows;
}

int launchMfmaFloatScan(const ScanArgs& scan, const PhaseArgs& phase, const EmitArgs& emit,
                        int workgroups, hipStream_t stream) {
    if (phase.items <= 0) {
        return ZCGVS_OK;
    }
    Launch launch{scan, phase, emit, workgroups, stream};
    if (!dispatchShape(scan.dtype, scan.dim, launch)) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: float MFMA scan does not take this shape");
    }
    return launch.status;
}

}  // namespace zcgvs_hip
