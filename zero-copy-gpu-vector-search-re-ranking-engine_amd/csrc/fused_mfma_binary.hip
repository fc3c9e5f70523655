// Binary (1-bit) MFMA fused scan: Hamming distances of sign-packed corpus rows to a batch of
// sign-packed queries on the fp4 matrix cores, with the threshold emission of fused.hpp. The
// reference computes popc(c ^ q) word by word on the VALU (src/cuda/similarity.cu:169-238,
// hammingScanKernel) and scores (d - 2h) / d (include/zcgvs/cuda/decode.cuh:45-47).
//
// Arithmetic. With r the row's bits and q the query's bits as 0/1 values,
//   sum_k r_k (1 - 2 q_k) = popc(r) - 2 r.q,  so  h = popc(r) + popc(q) - 2 r.q = acc / 2 + popc(q)
// where acc is the v_mfma_scale_f32_16x16x128_f8f6f4 product of the row's e2m1 nibbles (A: 0, 0.5,
// 1 or 2) with the query's (B: +-4, +-2 or +-1), chosen so that every product is 2 r_k (1 - 2 q_k)
// (spreadNibbles, signNibbles). Every value is a small integer (|acc| <= 2 d, far below 2^24), so
// the fp32 accumulator and h are exact; the score is the reference's IEEE division (d - 2h) / d.
// A threshold phase compares h itself with the integer threshold equivalent to the query's key
// threshold (scores are strictly decreasing in h), so the division runs only for keys that pass.
//
// Expansion. Each lane turns one 32-bit word of its row into 32 nibbles per k-step: nibble e of
// dword j holds bit 4e + j of the word. That is a fixed permutation of the word's dims, and the
// query's B operand uses the same one; a dot product does not depend on the order of its dims.
// Four ANDs and one shift per word, shared by the two query groups of 16 a wavefront serves. (An
// int8 form on v_mfma_i32_16x16x64_i8 takes two steps and eight ANDs per word for the same
// matrix-core cycles per step.)
//
// Work split. Launches of up to 32 queries (one set, two MFMA query groups of 16) run
// mfmaBinaryStreamKernel: each of 12 wavefronts holds the set's B operands in registers and
// streams its own rows through LDS slots of its own (no shared tile, no barrier). It serves the sketch plan of
// any batch, one launch per set: a sketch mode (the least distance of each query per pair of
// wavefronts, no keys) and a rerun mode (the device list of flagged queries). Larger batches scan
// up to 4 sets (128 queries) at a time on mfmaBinaryScanKernel: 12 wavefronts, three per SIMD,
// each with one set's B operands in registers, share the tiles below and split each tile's 16-row
// blocks among the wavefronts of a set. (Eight wavefronts serving two sets each, four query groups
// per row expansion, measured 1-16% slower: at 96 queries a third of their groups are empty.)
//
// MFMA layout (16x16x128, fp4 operands). Lane l supplies row (A) / query (B) l % 16 and 32 dims
// of lane group h = l / 16 per step: 16-byte chunk h + 4j of the row covers steps 4j .. 4j + 3,
// one word each; A and B use the same assignment, so every dim is counted once. D: lane l holds
// query l % 16 and rows 4h + i, i < 4.
//
// Corpus streaming as in the other MFMA scans (lds_copy.hpp): 48 KB tiles HBM -> LDS by
// global_load_lds_dwordx4 in a 3-deep ring (smaller tiles in deeper rings measured slower: the
// per-tile barrier costs more than the extra copies in flight gain). LDS slot s of row r holds chunk s ^ swz(r) with
// swz(r) = (r / (256 / row bytes)) & (chunks - 1), so the 16 rows of one ds_read_b128
// quarter-wave hit 16 distinct 16-byte bank groups.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.hpp"
#include "fused.hpp"
#include "lds_copy.hpp"

namespace zcgvs_hip {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 768;  // the tile kernel: 12 wavefronts
constexpr int kWaves = kThreads / kWave;
constexpr int kSetQueries = 32;  // two MFMA query groups of 16 per wavefront
constexpr int kQueriesPerLaunch = 4 * kSetQueries;
constexpr int kTileSetsPerWave = 1;  // query sets per tile-kernel wavefront
constexpr int kTileBytesTarget = 48 * 1024;
constexpr int kMinBatch = 4;  // below this the VALU popcount scan does less work per row

template <int kWords>
struct BinaryTile {
    static constexpr int kRowBytes = kWords * 4;
    static constexpr int kChunks = kRowBytes / 16;
    static constexpr int kLaneChunks = kChunks / 4;  // chunks per lane group
    static constexpr int kRows = kTileBytesTarget / kRowBytes;
    static constexpr int kRowBlocks = kRows / 16;
    static constexpr int kTileBytes = kRows * kRowBytes;
    static constexpr int kDepth = 3;
    static constexpr int kCopies = kTileBytes / 16 / kThreads;
    static constexpr int kRowsPerBankPeriod = 256 / kRowBytes;
    static_assert(kChunks % 4 == 0 && kChunks <= 8, "rows of 64 or 128 bytes (queries in registers)");
    static_assert(kTileBytes % (16 * kThreads) == 0, "tile must split over the lanes");
    static_assert((kDepth - 1) * kCopies < 63, "copies in flight fit the vmcnt counter");
    __host__ __device__ static constexpr int swizzle(int row) {
        return (row / kRowsPerBankPeriod) & (kChunks - 1);
    }
};

// fp4 (e2m1) operands: nibble 0001 is 0.5 (the format's one subnormal, which the matrix core takes
// exactly: the scans are bit-exact against the oracle), 0010 is 1, 0100 is 2, 0110 is 4 and bit 3
// is the sign. A row word becomes 32 nibbles: nibble e of dword j holds bit 4e + j of the word in
// place (j < 3: 0 or 0.5, 1, 2) or moved to nibble bit 2 (j = 3: 0 or 2), four ANDs and one shift.
__device__ __forceinline__ v4i spreadNibbles(std::uint32_t word) {
    v4i out;
    out[0] = static_cast<int>(word & 0x11111111u);
    out[1] = static_cast<int>(word & 0x22222222u);
    out[2] = static_cast<int>(word & 0x44444444u);
    out[3] = static_cast<int>((word >> 1) & 0x44444444u);
    return out;
}

// The same 32 dims of a query word as spreadNibbles, as (1 - 2 bit) times 4, 2, 1, 1 for j = 0..3,
// so that every product with spreadNibbles' nibble is 2 r (1 - 2 q).
__device__ __forceinline__ v4i signNibbles(std::uint32_t word) {
    v4i out;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const std::uint32_t magnitude = j == 0 ? 0x66666666u : (j == 1 ? 0x44444444u : 0x22222222u);
        out[j] = static_cast<int>((((word >> j) & 0x11111111u) << 3) | magnitude);
    }
    return out;
}

// v_mfma_scale_f32_16x16x128_f8f6f4 with both operands fp4 (format code 4; the instruction reads
// the low four registers of each) and unit scales (E8M0 127 = 2^0). Products of +-2 and their sums
// below 2^24 are exact in the fp32 accumulators.
__device__ __forceinline__ v4f mfmaNibbles(const v4i& a, const v4i& b, const v4f& c) {
    constexpr int kFp4 = 4;
    constexpr int kScaleOne = 127;
    const v8i a8 = __builtin_shufflevector(a, a, 0, 1, 2, 3, 0, 1, 2, 3);
    const v8i b8 = __builtin_shufflevector(b, b, 0, 1, 2, 3, 0, 1, 2, 3);
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a8, b8, c, kFp4, kFp4, 0, kScaleOne, 0, kScaleOne);
}

// The integer form of query q's key threshold in a threshold phase: a key passes when h < h_limit,
// or h == h_limit and its row is below row_limit (the lower index wins a tie); without a threshold
// every h passes.
template <int kDim>
__device__ __forceinline__ void binaryThreshold(const EmitArgs& emit, int q, int& h_limit, std::uint32_t& row_limit) {
    h_limit = kDim + 1;
    row_limit = 0xFFFFFFFFu;
    const std::uint64_t tau = emit.tau[q];
    if (tau != 0ull) {
        const float t_score = keyScore(tau);
        // the h whose score (d - 2h) / d is exactly the threshold's score
        const float estimate = (static_cast<float>(kDim) - t_score * static_cast<float>(kDim)) * 0.5f;
        int ht = estimate >= 0.0f && estimate <= static_cast<float>(kDim) ? static_cast<int>(rintf(estimate)) : 0;
        for (int c = max(0, ht - 2); c <= min(kDim, ht + 2); ++c) {
            if (static_cast<float>(kDim - 2 * c) / static_cast<float>(kDim) == t_score) {
                ht = c;
            }
        }
        h_limit = ht;
        row_limit = 0xFFFFFFFFu - static_cast<std::uint32_t>(tau);
    }
}

template <int kWords, bool kDense>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3, 3)))
void mfmaBinaryScanKernel(ScanArgs scan, PhaseArgs phase, EmitArgs emit, int q_offset, int q_count) {
    using Tile = BinaryTile<kWords>;
    constexpr int kRows = Tile::kRows;
    constexpr int kRowBytes = Tile::kRowBytes;
    constexpr int kChunks = Tile::kChunks;
    constexpr int kLaneChunks = Tile::kLaneChunks;
    constexpr int kSteps = kLaneChunks * 4;  // one word (32 dims) per lane and step, 128 per step
    constexpr int kDepth = Tile::kDepth;
    constexpr int kCopies = Tile::kCopies;
    constexpr int kRowBlocks = Tile::kRowBlocks;
    constexpr int kDim = kWords * 32;
    constexpr int kGroups = 2 * kTileSetsPerWave;  // query groups of 16 per wavefront

    __shared__ __attribute__((aligned(16))) std::uint8_t ring[kDepth][Tile::kTileBytes];
    __shared__ std::uint32_t lds_count[kQueriesPerLaunch];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // wave-uniform: scalar indexing
    const int r16 = lane & 15;
    const int h = lane >> 4;
    // wavefront sets of kTileSetsPerWave query sets each; the launch's wavefronts split among them
    const int wave_sets = (q_count + kTileSetsPerWave * kSetQueries - 1) / (kTileSetsPerWave * kSetQueries);
    const int waves_per_set = kWaves / wave_sets;
    const bool wave_active = wave < wave_sets * waves_per_set;
    const int wave_set = wave % wave_sets;
    const int first_block = wave / wave_sets;
    const int first_query = wave_set * kTileSetsPerWave * kSetQueries;
    bool live[kGroups];  // the group has queries (wave-uniform)
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
        live[g] = first_query + g * 16 < q_count;
    }
    const long long doc_count = scan.doc_count;
    const std::uint8_t* corpus = static_cast<const std::uint8_t*>(scan.corpus);
    const std::uint32_t* qwords = static_cast<const std::uint32_t*>(scan.queries);

    // ---- per query group g of the wavefront: B operands, popc(q), integer threshold ----
    v4i qb[kGroups][kSteps];
    int popq[kGroups];
    int q_of[kGroups];
    bool valid_of[kGroups];
    int h_limit[kGroups];  // keys pass when h < h_limit, or h == h_limit and row < row_limit
    std::uint32_t row_limit[kGroups];
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
        const int qlocal = first_query + g * 16 + r16;
        valid_of[g] = wave_active && qlocal < q_count;
        const int q = q_offset + min(qlocal, q_count - 1);
        q_of[g] = q;
        const std::uint32_t* qrow = qwords + static_cast<std::size_t>(q) * kWords;
        u32x4 chunk[kLaneChunks];
#pragma unroll
        for (int jc = 0; jc < kLaneChunks; ++jc) {
            chunk[jc] = *reinterpret_cast<const u32x4*>(qrow + 4 * (h + 4 * jc));
        }
        int pop = 0;
#pragma unroll
        for (int jc = 0; jc < kLaneChunks; ++jc) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                pop += __popc(chunk[jc][w]);
            }
        }
        // the four lane groups hold disjoint chunks of the query
        pop += waveXor(pop, 16);
        pop += waveXor(pop, 32);
        popq[g] = pop;
#pragma unroll
        for (int t = 0; t < kSteps; ++t) {
            qb[g][t] = valid_of[g] ? signNibbles(chunk[t / 4][t % 4]) : v4i{0, 0, 0, 0};
        }
        h_limit[g] = kDim + 1;  // no threshold: every h passes
        row_limit[g] = 0xFFFFFFFFu;
        if constexpr (!kDense) {
            binaryThreshold<kDim>(emit, q, h_limit[g], row_limit[g]);
        }
    }
    // acc threshold of the fast reject (acc = 2 (h - popc(q)); invalid queries never pass)
    float acc_limit[kGroups];
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
        acc_limit[g] = static_cast<float>(2 * (valid_of[g] ? h_limit[g] - popq[g] : -(kDim + 1)));
    }
    for (int i = tid; i < kQueriesPerLaunch; i += kThreads) {
        lds_count[i] = 0u;
    }

    // ---- copy plan ----
    std::uint32_t copy_off[kCopies];
#pragma unroll
    for (int i = 0; i < kCopies; ++i) {
        const int p = (wave * kCopies + i) * kWave + lane;
        const int row = p / kChunks;
        const int slot = p - row * kChunks;
        copy_off[i] = static_cast<std::uint32_t>(row * kRowBytes + (slot ^ Tile::swizzle(row)) * 16);
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
            const int last = static_cast<int>(doc_count - row0) - 1;
#pragma unroll
            for (int i = 0; i < kCopies; ++i) {
                const int row = static_cast<int>(copy_off[i]) / kRowBytes;
                const std::uint32_t off = copy_off[i] - static_cast<std::uint32_t>((row - min(row, last)) * kRowBytes);
                copyToLds(base, off, __builtin_amdgcn_readfirstlane(slot_base + (wave * kCopies + i) * kWave * 16));
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
        waitTiles<kCopies, kDepth - 2>(later);
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");  // no LDS access moves above the barrier
    };

    // chunk h + 4 jc of row r16 of a block
    std::uint32_t a_off[kLaneChunks];
#pragma unroll
    for (int jc = 0; jc < kLaneChunks; ++jc) {
        a_off[jc] = static_cast<std::uint32_t>(r16 * kRowBytes + ((h + 4 * jc) ^ Tile::swizzle(r16)) * 16);
    }

    auto emitKeys = [&](const v4f& acc, int g, long long row0, int block, long long item_) {
        if (!valid_of[g]) {
            return;
        }
        const int q = q_of[g];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int local = block * 16 + 4 * h + i;
            const long long row = row0 + local;
            const int hd = (static_cast<int>(acc[i]) >> 1) + popq[g];  // acc = 2 (h - popc(q)), exactly
            if constexpr (kDense) {
                std::uint64_t key = 0ull;
                if (row < doc_count) {
                    const float score = static_cast<float>(kDim - 2 * hd) / static_cast<float>(kDim);
                    key = makeKey(score, static_cast<std::uint32_t>(row));
                }
                emit.dense[static_cast<std::size_t>(q) * emit.dense_stride + item_ * kRows + local] = key;
            } else {
                const std::uint32_t r32 = static_cast<std::uint32_t>(row);
                const bool pass = hd < h_limit[g] || (hd == h_limit[g] && r32 < row_limit[g]);
                if (pass && row < doc_count) {
                    const float score = static_cast<float>(kDim - 2 * hd) / static_cast<float>(kDim);
                    appendCandidate(emit, lds_count, q, q_offset, scan.batch, makeKey(score, r32));
                }
            }
        }
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
            for (int block = first_block; block < kRowBlocks; block += waves_per_set) {
                const std::uint8_t* rows = ring[slot] + block * 16 * kRowBytes;
                u32x4 chunk[kLaneChunks];
#pragma unroll
                for (int jc = 0; jc < kLaneChunks; ++jc) {
                    chunk[jc] = *reinterpret_cast<const u32x4*>(rows + a_off[jc]);
                }
                v4f acc[kGroups];
#pragma unroll
                for (int g = 0; g < kGroups; ++g) {
                    acc[g] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
                }
                // One path for any number of live query groups (a group without queries has zero
                // B operands), so the compiler has no several copies of the expansion to hoist;
                // each expansion feeds every group's MFMA. The A operand is double-buffered: step
                // t's MFMAs are issued first, then step t + 1's expansion into the other buffer,
                // which the matrix core is not reading, so the VALU work runs under the MFMAs
                // instead of waiting for them to read their operands; a sched_barrier per step pins
                // that order.
                v4i a[2];
                a[0] = spreadNibbles(chunk[0][0]);
#pragma unroll
                for (int t = 0; t < kSteps; ++t) {
#pragma unroll
                    for (int g = 0; g < kGroups; ++g) {
                        acc[g] = mfmaNibbles(a[t % 2], qb[g][t], acc[g]);
                    }
                    if (t + 1 < kSteps) {
                        a[(t + 1) % 2] = spreadNibbles(chunk[(t + 1) / 4][(t + 1) % 4]);
                        // keeps step t's operand allocated until the expansion is written, so
                        // the two buffers never share registers
                        asm volatile("" ::"v"(a[t % 2]));
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                if constexpr (kDense) {
#pragma unroll
                    for (int g = 0; g < kGroups; ++g) {
                        if (live[g]) {
                            emitKeys(acc[g], g, row0, block, item);
                        }
                    }
                } else {
                    // Fast reject: a key can pass only if acc <= 2 (h_limit - popc(q)) (h = acc / 2 +
                    // popc(q)); one ballot over the wavefront's products usually ends here.
                    bool maybe = false;
#pragma unroll
                    for (int g = 0; g < kGroups; ++g) {
                        const float m = fminf(fminf(acc[g][0], acc[g][1]), fminf(acc[g][2], acc[g][3]));
                        maybe = maybe || m <= acc_limit[g];
                    }
                    if (__builtin_amdgcn_ballot_w64(maybe) != 0) {
#pragma unroll
                        for (int g = 0; g < kGroups; ++g) {
                            if (live[g]) {
                                emitKeys(acc[g], g, row0, block, item);
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

constexpr int kStreamThreads = 768;
constexpr int kStreamWaves = kStreamThreads / kWave;
constexpr int kStreamSlots = 3;  // LDS pair slots per wavefront

// One query set (<= 32 queries): each of the workgroup's 12 wavefronts (three per SIMD) holds the
// set's B operands in registers and streams its own rows, 32 rows (two 16-row blocks) at a time,
// through three LDS pair slots of its own (144 KB per workgroup at 1024 bits): global_load_lds
// copies of whole cache lines land a pair three pairs ahead, and the pair being multiplied is read
// from its slot into registers in the MFMA layout. No tile is shared, so there is no barrier in
// the loop. (Loading the MFMA layout straight into registers reads half cache lines per
// quarter-wave: measured 8% slower for 50M x 1024, B = 32; 16 wavefronts with the B operands in
// LDS and two slots each, 1.5-2% slower.) Each B operand feeds two MFMAs (the pair's two blocks).
// Wavefront w of workgroup b takes pairs w * gridDim.x + b, + 12 * gridDim.x, ... of the phase's
// items (an item's pairs in order), so the pairs spread over the workgroups first.
//
// Modes: kStreamThreshold (keys above the threshold to the workgroup's segment), kStreamDense
// (every key to its fixed slot), kStreamSketch (no keys: per pair of wavefronts the least Hamming
// distance of each query, as a score, to sketch slot 6 * workgroup + wave / 2) and kStreamRerun
// (kStreamThreshold over the queries of EmitArgs::q_list, in the list's segment layout; a kernel
// of its own, so profiles tell the fallback's launches apart).
constexpr int kStreamThreshold = 0;
constexpr int kStreamDense = 1;
constexpr int kStreamSketch = 2;
constexpr int kStreamRerun = 3;
constexpr int kStreamSketchSlots = kStreamWaves / 2;  // per workgroup

template <int kWords, int kMode>
__global__ __launch_bounds__(kStreamThreads)
void mfmaBinaryStreamKernel(ScanArgs scan, PhaseArgs phase, EmitArgs emit, int q_offset, int q_count) {
    constexpr bool kDense = kMode == kStreamDense;
    constexpr bool kSketch = kMode == kStreamSketch;
    constexpr bool kListed = kMode == kStreamRerun;
    using Tile = BinaryTile<kWords>;
    constexpr int kRows = Tile::kRows;
    constexpr int kRowBytes = Tile::kRowBytes;
    constexpr int kLaneChunks = Tile::kLaneChunks;
    constexpr int kSteps = kLaneChunks * 4;  // one word (32 dims) per lane and step, 128 per step
    constexpr int kPairs = Tile::kRowBlocks / 2;
    constexpr int kDim = kWords * 32;
    static_assert(Tile::kRowBlocks % 2 == 0, "an item splits into 32-row pairs");

    constexpr int kChunks = Tile::kChunks;
    constexpr int kPairBytes = 32 * kRowBytes;
    constexpr int kPairCopies = kPairBytes / 1024;  // one 1 KB global_load_lds_dwordx4 per 1024 / kRowBytes rows
    constexpr int kRowsPerCopy = 1024 / kRowBytes;
    // each wavefront's two pair slots; slot position s of pair row r holds chunk s ^ swizzle(r)
    __shared__ __attribute__((aligned(16))) std::uint8_t pair_lds[kStreamWaves][kStreamSlots][kPairBytes];
    __shared__ std::uint32_t lds_count[kSetQueries];
    __shared__ int lds_sketch[kSketch ? kStreamWaves : 1][kSetQueries];

    // A rerun scans list entries [q_offset, q_offset + q_count) of q_list, of which
    // F = *q_list_count exist (uniform over the launch, so a workgroup past them returns at once).
    int seg_batch = scan.batch;
    int seg_log2 = emit.seg_log2;
    if constexpr (kListed) {
        const int entries = static_cast<int>(__builtin_amdgcn_readfirstlane(*emit.q_list_count));
        if (entries <= q_offset) {
            return;
        }
        q_count = min(q_count, entries - q_offset);
        seg_batch = entries;
        seg_log2 = rerunSegLog2(emit.seg_log2, scan.batch, entries);
    }
    // the query of launch-local query `local` (a rerun's list entry q_offset + local)
    auto queryOf = [&](int local) {
        if constexpr (kListed) {
            return static_cast<int>(emit.q_list[q_offset + local]);
        }
        return q_offset + local;
    };

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    // wave-uniform (a scalar register), so the pair indexing below runs on the scalar unit
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int r16 = lane & 15;
    const int h = lane >> 4;
    const bool two_groups = 16 < q_count;  // launch-uniform
    const long long doc_count = scan.doc_count;
    const std::uint8_t* corpus = static_cast<const std::uint8_t*>(scan.corpus);
    const std::uint32_t* qwords = static_cast<const std::uint32_t*>(scan.queries);

    // B operands: lane l of group g at step t supplies query g * 16 + l % 16, word t % 4 of its
    // chunk l / 16 + 4 (t / 4) (as the A operand's lanes do for their rows)
    v4i qreg[kSteps][2];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
        const int qlocal = g * 16 + r16;
#pragma unroll
        for (int t = 0; t < kSteps; ++t) {
            v4i value = {0, 0, 0, 0};
            if (qlocal < q_count) {
                const std::uint32_t word = qwords[static_cast<std::size_t>(queryOf(qlocal)) * kWords +
                                                  4 * (h + 4 * (t / 4)) + t % 4];
                value = signNibbles(word);
            }
            qreg[t][g] = value;
        }
    }
    for (int i = tid; i < kSetQueries; i += kStreamThreads) {
        lds_count[i] = 0u;
    }
    // this lane's two queries (column r16 of each group's D): popc(q) and the integer threshold
    int popq[2];
    int q_of[2];
    bool valid_of[2];
    int h_limit[2];
    std::uint32_t row_limit[2];
    float acc_limit[2];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
        const int qlocal = g * 16 + r16;
        valid_of[g] = qlocal < q_count;
        const int q = queryOf(min(qlocal, q_count - 1));
        q_of[g] = q;
        const std::uint32_t* qrow = qwords + static_cast<std::size_t>(q) * kWords;
        // the four lane groups hold disjoint chunks h + 4 jc of the query
        int pop = 0;
#pragma unroll
        for (int jc = 0; jc < kLaneChunks; ++jc) {
            const u32x4 words = *reinterpret_cast<const u32x4*>(qrow + 4 * (h + 4 * jc));
            pop += __popc(words[0]) + __popc(words[1]) + __popc(words[2]) + __popc(words[3]);
        }
        pop += waveXor(pop, 16);
        pop += waveXor(pop, 32);
        popq[g] = pop;
        h_limit[g] = kDim + 1;
        row_limit[g] = 0xFFFFFFFFu;
        if constexpr (!kDense && !kSketch) {
            binaryThreshold<kDim>(emit, q, h_limit[g], row_limit[g]);
        }
        acc_limit[g] = static_cast<float>(2 * (valid_of[g] ? h_limit[g] - popq[g] : -(kDim + 1)));
    }
    __syncthreads();
    int best_hd[2] = {kDim + 1, kDim + 1};  // sketch: the lane's least distance per query group

    // acc holds 2 (popc(r) - 2 r.q) exactly, so h = acc / 2 + popc(q)
    auto distance = [&](float acc, int g) { return (static_cast<int>(acc) >> 1) + popq[g]; };
    auto emitKeys = [&](const v4f& acc, int g, long long row0, int local0, long long item_) {
        if (!valid_of[g]) {
            return;
        }
        const int q = q_of[g];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int local = local0 + 4 * h + i;  // row within the item
            const long long row = row0 + local;
            const int hd = distance(acc[i], g);
            if constexpr (kDense) {
                std::uint64_t key = 0ull;
                if (row < doc_count) {
                    const float score = static_cast<float>(kDim - 2 * hd) / static_cast<float>(kDim);
                    key = makeKey(score, static_cast<std::uint32_t>(row));
                }
                emit.dense[static_cast<std::size_t>(q) * emit.dense_stride + item_ * kRows + local] = key;
            } else {
                const std::uint32_t r32 = static_cast<std::uint32_t>(row);
                const bool pass = hd < h_limit[g] || (hd == h_limit[g] && r32 < row_limit[g]);
                if (pass && row < doc_count) {
                    const float score = static_cast<float>(kDim - 2 * hd) / static_cast<float>(kDim);
                    // to this workgroup's segment of the launch's query g * 16 + r16
                    const int qlocal = g * 16 + r16;
                    const std::uint32_t slot = atomicAdd(&lds_count[qlocal], 1u);
                    if (slot < (1u << seg_log2)) {
                        emit.seg[((static_cast<std::size_t>(blockIdx.x) * seg_batch + q_offset + qlocal) << seg_log2) +
                                 slot] = makeKey(score, r32);
                    }
                }
            }
        }
    };
    // Pair p's rows into LDS slot `slot` of this wavefront: copy k moves pair rows
    // k * kRowsPerCopy .. + kRowsPerCopy - 1, lane l the 16 bytes of row k * kRowsPerCopy + l / kChunks
    // that land at slot position l % kChunks, so every copy reads 1 KB of consecutive rows (whole
    // cache lines per quarter-wave). Rows past the corpus re-read its last row (their keys are never
    // emitted). Pair indices stay below 2^31: 32-bit division by the constant kPairs.
    // copy_offset[k]: this lane's source byte offset within the pair for copy k
    std::uint32_t copy_offset[kPairCopies];
#pragma unroll
    for (int k = 0; k < kPairCopies; ++k) {
        const int r = k * kRowsPerCopy + lane / kChunks;
        copy_offset[k] = static_cast<std::uint32_t>(r * kRowBytes + ((lane % kChunks) ^ Tile::swizzle(r)) * 16);
    }
    auto copyPair = [&](long long p, int slot) {
        const std::uint32_t p32 = static_cast<std::uint32_t>(p);
        const std::uint32_t it = p32 / kPairs;
        const long long row0 = phaseBlock(it, phase.stride, phase.skip) * kRows + 32 * static_cast<int>(p32 - it * kPairs);
        const std::uint32_t base = ldsAddress(&pair_lds[wave][slot][0]);
        if (row0 + 32 <= doc_count) {
            // a whole pair: a wave-uniform base and the lane's fixed offsets
            const std::uint8_t* pair_base = corpus + static_cast<std::size_t>(row0) * kRowBytes;
#pragma unroll
            for (int k = 0; k < kPairCopies; ++k) {
                copyToLds(pair_base, copy_offset[k], base + k * 1024);
            }
        } else {
#pragma unroll
            for (int k = 0; k < kPairCopies; ++k) {
                const int r = k * kRowsPerCopy + lane / kChunks;
                const long long row = min(row0 + r, doc_count - 1);
                copyToLds(corpus + static_cast<std::size_t>(row) * kRowBytes + (copy_offset[k] - r * kRowBytes),
                          base + k * 1024);
            }
        }
    };
    // The lane's A chunks of a staged pair: row 16 b + r16, chunk h + 4 jc (the 16 rows of one
    // ds_read_b128 quarter-wave hit 16 distinct 16-byte bank groups through the swizzle).
    auto readPair = [&](int slot, u32x4 (&dst)[2][kLaneChunks]) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int r = 16 * b + r16;
#pragma unroll
            for (int jc = 0; jc < kLaneChunks; ++jc) {
                const int position = (h + 4 * jc) ^ Tile::swizzle(r);
                dst[b][jc] = *reinterpret_cast<const u32x4*>(&pair_lds[wave][slot][r * kRowBytes + position * 16]);
            }
        }
    };
    auto processPair = [&](const u32x4 (&cur)[2][kLaneChunks], long long p) {
        // the pair's rows first: phaseBlock branches, and products computed before a branch whose
        // far side uses them would be sunk past it, out of the step-by-step schedule below
        const std::uint32_t p32 = static_cast<std::uint32_t>(p);
        const std::uint32_t it = p32 / kPairs;
        const long long row0 = phaseBlock(it, phase.stride, phase.skip) * kRows;
        const int pair_row = 32 * static_cast<int>(p32 - it * kPairs);
        v4f acc[2][2] = {};
        v4i a[2];
        a[0] = spreadNibbles(cur[0][0][0]);
        a[1] = spreadNibbles(cur[1][0][0]);
        // The B operands of step t + 1 are read from LDS during step t. The lane's index is
        // opaque to the compiler, which would otherwise keep every step's B operands in registers
        // across pairs (64 more registers, and spills).
#pragma unroll
        for (int t = 0; t < kSteps; ++t) {
            const v4i b0 = qreg[t][0];
            const v4i b1 = qreg[t][1];
            acc[0][0] = mfmaNibbles(a[0], b0, acc[0][0]);
            acc[0][1] = mfmaNibbles(a[0], b1, acc[0][1]);
            acc[1][0] = mfmaNibbles(a[1], b0, acc[1][0]);
            acc[1][1] = mfmaNibbles(a[1], b1, acc[1][1]);
            if (t + 1 < kSteps) {
                a[0] = spreadNibbles(cur[0][(t + 1) / 4][(t + 1) % 4]);
                a[1] = spreadNibbles(cur[1][(t + 1) / 4][(t + 1) % 4]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // every product is finished here: block 1's are otherwise sunk past block 0's emission,
        // keeping its operands live across it
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            asm volatile("" : "+v"(acc[b][0]), "+v"(acc[b][1]));
        }
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            if constexpr (kSketch) {
                // the least distance over the lane's rows that exist (rows past the corpus
                // re-read its last row)
#pragma unroll
                for (int g = 0; g < 2; ++g) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const long long row = row0 + pair_row + 16 * b + 4 * h + i;
                        const int hd = distance(acc[b][g][i], g);
                        best_hd[g] = row < doc_count ? min(best_hd[g], hd) : best_hd[g];
                    }
                }
            } else if constexpr (kDense) {
                emitKeys(acc[b][0], 0, row0, pair_row + 16 * b, it);
                if (two_groups) {
                    emitKeys(acc[b][1], 1, row0, pair_row + 16 * b, it);
                }
            } else {
                // fast reject: a key can pass only if acc <= 2 (h_limit - popc(q))
                const float m0 = fminf(fminf(acc[b][0][0], acc[b][0][1]), fminf(acc[b][0][2], acc[b][0][3]));
                const float m1 = fminf(fminf(acc[b][1][0], acc[b][1][1]), fminf(acc[b][1][2], acc[b][1][3]));
                if (__builtin_amdgcn_ballot_w64(m0 <= acc_limit[0] || m1 <= acc_limit[1]) != 0) {
                    emitKeys(acc[b][0], 0, row0, pair_row + 16 * b, it);
                    if (two_groups) {
                        emitKeys(acc[b][1], 1, row0, pair_row + 16 * b, it);
                    }
                }
            }
        }
    };

    const long long pairs = phase.items * kPairs;
    const long long stride = static_cast<long long>(gridDim.x) * kStreamWaves;
    // workgroup-first: with few pairs every workgroup (candidate segment) still gets its share
    long long p = static_cast<long long>(wave) * gridDim.x + blockIdx.x;
    // Three pairs in flight while one is multiplied, with no registers held for them: pair i waits
    // in slot i % 3 of the wavefront's LDS, copied there three pairs ahead. Every iteration issues
    // one pair's copies (past the phase's end, its last pair again), so before pair i is read only
    // pairs i + 1 and i + 2 may still be pending (later global stores of the emission only make
    // the wait stricter). The copies are inline assembly the compiler does not count, hence the
    // explicit waits; the memory clobbers keep the LDS reads between them.
    const long long mine = p < pairs ? (pairs - p + stride - 1) / stride : 0;  // this wave's pairs
    if (mine > 0) {
        copyPair(p, 0);
        copyPair(min(p + stride, pairs - 1), 1);
        copyPair(min(p + 2 * stride, pairs - 1), 2);
    }
    for (long long i = 0; i < mine; ++i) {
        const int slot = static_cast<int>(i % 3);
        asm volatile("s_waitcnt vmcnt(%0)" : : "n"(2 * kPairCopies) : "memory");
        u32x4 cur[2][kLaneChunks];
        readPair(slot, cur);
        // the slot's reads are done before its next copy is issued
        asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
        copyPair(min(p + 3 * stride, pairs - 1), slot);
        processPair(cur, p);
        p += stride;
    }
    // no copy may land in LDS after the wavefront ends
    asm volatile("s_waitcnt vmcnt(0)" : : : "memory");

    if constexpr (kSketch) {
        // the least distance per query over the lane groups h, then over each pair of
        // wavefronts, written as a score to slot 6 * workgroup + wave / 2
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            best_hd[g] = min(best_hd[g], waveXor(best_hd[g], 16));
            best_hd[g] = min(best_hd[g], waveXor(best_hd[g], 32));
        }
        if (h == 0) {
            lds_sketch[wave][r16] = best_hd[0];
            lds_sketch[wave][16 + r16] = best_hd[1];
        }
        __syncthreads();
        for (int i = tid; i < kStreamSketchSlots * q_count; i += kStreamThreads) {
            const int pair = i / q_count;
            const int local = i - pair * q_count;
            const int hd = min(lds_sketch[2 * pair][local], lds_sketch[2 * pair + 1][local]);
            const float score =
                hd <= kDim ? static_cast<float>(kDim - 2 * hd) / static_cast<float>(kDim) : -INFINITY;
            const std::size_t slot = static_cast<std::size_t>(kStreamSketchSlots) * blockIdx.x + pair;
            emit.sketch[slot * scan.batch + q_offset + local] = score;
        }
        return;
    }
    if constexpr (!kDense) {
        __syncthreads();
        for (int i = tid; i < q_count; i += kStreamThreads) {
            emit.seg_count[static_cast<std::size_t>(blockIdx.x) * seg_batch + q_offset + i] = lds_count[i];
        }
    }
}

template <int kWords>
int launchShape(const ScanArgs& scan, const PhaseArgs& phase, const EmitArgs& emit, int workgroups,
                hipStream_t stream) {
    const long long wanted = phase.dense ? std::min<long long>(phase.items, workgroups) : workgroups;
    const dim3 grid(static_cast<unsigned>(std::max(1LL, wanted)));
    // sketch and rerun launches always stream, set by set; threshold, dense and full scans of more
    // than one set run the tile kernel, which reads each row once for up to four sets (at 48 and 64
    // queries 1.89 and 2.03 ms per step against 2.33 streaming set by set, 50M x 1024)
    const bool streamed = scan.batch <= kSetQueries || phase.sketch != 0 || emit.q_list != nullptr;
    const int per_launch = streamed ? kSetQueries : kQueriesPerLaunch;
    for (int q0 = 0; q0 < scan.batch; q0 += per_launch) {
        const int count = std::min(per_launch, scan.batch - q0);
        if (count <= kSetQueries) {
            // one query set: the streaming kernel
            if (phase.dense) {
                mfmaBinaryStreamKernel<kWords, kStreamDense>
                    <<<grid, kStreamThreads, 0, stream>>>(scan, phase, emit, q0, count);
            } else if (phase.sketch) {
                mfmaBinaryStreamKernel<kWords, kStreamSketch>
                    <<<grid, kStreamThreads, 0, stream>>>(scan, phase, emit, q0, count);
            } else if (emit.q_list != nullptr) {
                mfmaBinaryStreamKernel<kWords, kStreamRerun>
                    <<<grid, kStreamThreads, 0, stream>>>(scan, phase, emit, q0, count);
            } else {
                mfmaBinaryStreamKernel<kWords, kStreamThreshold>
                    <<<grid, kStreamThreads, 0, stream>>>(scan, phase, emit, q0, count);
            }
        } else if (phase.sketch || emit.q_list != nullptr) {
            return setError(ZCGVS_ERR_RUNTIME, "zcgvs: the binary tile scan has no sketch or rerun mode");
        } else if (phase.dense) {
            mfmaBinaryScanKernel<kWords, true><<<grid, kThreads, 0, stream>>>(scan, phase, emit, q0, count);
        } else {
            mfmaBinaryScanKernel<kWords, false><<<grid, kThreads, 0, stream>>>(scan, phase, emit, q0, count);
        }
        ZCGVS_LAUNCH_CHECK("binary mfma scan");
    }
    return ZCGVS_OK;
}

}  // namespace

bool mfmaBinarySupported(const ScanArgs& scan) {
    if (scan.dtype != ZCGVS_DTYPE_BINARY || scan.mask != nullptr || scan.lexical != nullptr ||
        scan.batch < kMinBatch) {
        return false;
    }
    if (!aligned16(scan.corpus) || !aligned16(scan.queries)) {
        return false;
    }
    return scan.dim == 512 || scan.dim == 1024;
}

bool mfmaBinaryStreams(const ScanArgs& scan) { return scan.dtype == ZCGVS_DTYPE_BINARY; }

int mfmaBinarySketchSlotsPerWorkgroup() { return kStreamSketchSlots; }

int mfmaBinaryBlockRows(const ScanArgs& scan) {
    return scan.dim == 512 ? BinaryTile<16>::kRows : BinaryTile<32>::kRows;
}

int launchMfmaBinaryScan(const ScanArgs& scan, const PhaseArgs& phase, const EmitArgs& emit,
                         int workgroups, hipStream_t stream) {
    if (phase.items <= 0) {
        return ZCGVS_OK;
    }
    switch (scan.dim) {
        case 512: return launchShape<16>(scan, phase, emit, workgroups, stream);
        case 1024: return launchShape<32>(scan, phase, emit, workgroups, stream);
        default:
            return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: binary MFMA scan does not take this shape");
    }
}

}  // namespace zcgvs_hip
