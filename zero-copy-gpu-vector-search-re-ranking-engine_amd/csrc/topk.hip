// Top-k selection: zcgvs_launch_topk (src/cuda/topk.cu:132-189 launchTopK) over a materialized
// [batch, doc_count] score matrix, and the per-query candidate merge used by the fused search.
//
// The reference sorts 1024-score tiles with a bitonic network and merges tile winners
// recursively; ties fall wherever the network puts them. Here the selection is an exact radix
// select on unique 64-bit keys (select.hpp), so the result is the stable (score desc, index asc)
// order of tests/cpp/cpu_reference.hpp:26-34 on every run. zcgvs_launch_topk reads the scores
// once: each block selects the best k of a tile of 8192-16384 scores in LDS, and one block per
// query merges the tile winners (two launches, no host round trip, capture safe).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.hpp"
#include "merge.hpp"
#include "select.hpp"

namespace zcgvs_hip {

namespace {

constexpr int kTileSize = 1024;      // reference tile (topk.cu:17), kept for the sizing helpers
constexpr int kMergeTile = 4096;     // reference merge tile (topk.cu:18)
constexpr int kMinScratchElements = 16 + kSelectBins + 16;
constexpr int kTopkTileMax = 16384;  // scores one block of zcgvs_launch_topk selects from (128 KB of keys)

// Scores per tile of zcgvs_launch_topk: the smallest of 8192, 12288 and 16384 whose tile winners (k
// per tile) fit the merge's LDS gather; 16384 when none does (the merge then reads the winners
// from global memory).
long long topkTileScores(long long doc_count, int k) {
    for (const long long tile : {8192LL, 12288LL, static_cast<long long>(kTopkTileMax)}) {
        if ((doc_count + tile - 1) / tile * k <= static_cast<long long>(kSelectLdsKeys)) {
            return tile;
        }
    }
    return kTopkTileMax;
}

// LDS of ldsSelectCut.
struct LdsSelect {
    std::uint32_t hist[kSelectBins];
    std::uint32_t scan[kMergeThreads / kWave];
    std::uint64_t wave_lo[kMergeThreads / kWave];
    std::uint64_t wave_hi[kMergeThreads / kWave];
    SelectState state;
    std::uint32_t count;
};

// The best min(k, n) of the n unique non-zero keys keys[0..n) (in LDS) by radix passes over them
// (select.hpp), run by a whole block of kMergeThreads threads; lo and hi are the calling thread's
// smallest and largest key (the passes start below the bits all keys share). Returns the cut:
// exactly min(k, n) keys are >= it (1 when n <= k). Ends with a barrier.
__device__ std::uint64_t ldsSelectCut(const std::uint64_t* keys, std::uint32_t n, int k, std::uint64_t lo,
                                      std::uint64_t hi, LdsSelect& lds) {
    const int t = threadIdx.x;
    lo = waveReduce64(lo, [](std::uint64_t x, std::uint64_t y) { return min(x, y); });
    hi = waveReduce64(hi, [](std::uint64_t x, std::uint64_t y) { return max(x, y); });
    if ((t & (kWave - 1)) == 0) {
        lds.wave_lo[t / kWave] = lo;
        lds.wave_hi[t / kWave] = hi;
    }
    __syncthreads();
    if (t < kWave) {
        constexpr int kSlots = kMergeThreads / kWave;
        std::uint64_t l = t < kSlots ? lds.wave_lo[t] : ~0ull;
        std::uint64_t h = t < kSlots ? lds.wave_hi[t] : 0ull;
        l = waveReduce64(l, [](std::uint64_t x, std::uint64_t y) { return min(x, y); });
        h = waveReduce64(h, [](std::uint64_t x, std::uint64_t y) { return max(x, y); });
        if (t == 0) {
            lds.state.prefix = 0ull;
            lds.state.bits = 0u;
            lds.state.need = min(n, static_cast<std::uint32_t>(k));
            lds.state.done = n <= static_cast<std::uint32_t>(k) ? 1u : 0u;
            if (n > static_cast<std::uint32_t>(k)) {  // at least two distinct keys
                const int common = __clzll(h ^ l);
                lds.state.prefix = common == 0 ? 0ull : (h >> (64 - common));
                lds.state.bits = static_cast<std::uint32_t>(common);
            }
        }
    }
    __syncthreads();
    for (int pass = 0; pass < kSelectPasses && !lds.state.done; ++pass) {
        const int width = min(11, 64 - static_cast<int>(lds.state.bits));
        for (int i = t; i < (1 << width); i += blockDim.x) {
            lds.hist[i] = 0u;
        }
        __syncthreads();
        const std::uint32_t bits = lds.state.bits;
        const std::uint64_t prefix = lds.state.prefix;
        const int shift = 64 - static_cast<int>(bits) - width;
        const std::uint64_t digit_mask = (1ull << width) - 1ull;
        for (std::uint32_t i = static_cast<std::uint32_t>(t); i < n; i += blockDim.x) {
            const std::uint64_t key = keys[i];
            if (bits == 0u || (key >> (64 - bits)) == prefix) {
                atomicAdd(&lds.hist[(key >> shift) & digit_mask], 1u);
            }
        }
        __syncthreads();
        selectPickBucket<kMergeThreads>(lds.hist, width, &lds.state, lds.scan);  // (ends with a barrier)
    }
    return n <= static_cast<std::uint32_t>(k) ? 1ull : selectThreshold(lds.state);
}

// Appends the keys of keys[0..n) that are >= cut to out[0..) (one slot reservation per wavefront
// step through lds.count, which the caller zeroes before a barrier), keeping at most `room`.
__device__ void ldsCollect(const std::uint64_t* keys, std::uint32_t n, std::uint64_t cut, std::uint64_t* out,
                           std::uint32_t room, LdsSelect& lds) {
    const int t = threadIdx.x;
    for (std::uint32_t base = 0; base < n; base += blockDim.x) {
        const std::uint32_t i = base + static_cast<std::uint32_t>(t);
        const std::uint64_t key = i < n ? keys[i] : 0ull;
        const bool take = key != 0ull && key >= cut;
        const std::uint64_t mask = __builtin_amdgcn_ballot_w64(take);
        if (mask != 0ull) {
            std::uint32_t slot0 = 0u;
            if ((t & (kWave - 1)) == 0) {
                slot0 = atomicAdd(&lds.count, static_cast<std::uint32_t>(__builtin_popcountll(mask)));
            }
            slot0 = __builtin_amdgcn_readfirstlane(slot0);
            const std::uint32_t slot = slot0 + __builtin_amdgcn_mbcnt_hi(static_cast<std::uint32_t>(mask >> 32),
                                                                         __builtin_amdgcn_mbcnt_lo(static_cast<std::uint32_t>(mask), 0u));
            if (take && slot < room) {
                out[slot] = key;
            }
        }
    }
}

// Block (t, q) of zcgvs_launch_topk: the keys of scores [t * tile, t * tile + n) of query q
// (n <= tile) go to LDS, their best min(k, n) are found by radix passes over the LDS keys
// (select.hpp), and written, in no particular order, to winners[q * stride + t * k + 0..k); the
// rest of the k slots get key 0 (no candidate).
__global__ __launch_bounds__(kMergeThreads) void topkTileKernel(const float* __restrict__ scores, int doc_count,
                                                                int tile, int k, std::uint64_t* __restrict__ winners,
                                                                std::size_t stride) {
    __shared__ std::uint64_t lds_keys[kTopkTileMax];
    __shared__ LdsSelect lds;

    const int t = threadIdx.x;
    const int q = blockIdx.y;
    const long long first = static_cast<long long>(blockIdx.x) * tile;
    std::uint64_t* out = winners + static_cast<std::size_t>(q) * stride + static_cast<std::size_t>(blockIdx.x) * k;
    if (first >= doc_count) {  // a padding tile of the group layout: no candidates
        for (int i = t; i < k; i += blockDim.x) {
            out[i] = 0ull;
        }
        return;
    }
    const std::uint32_t n = static_cast<std::uint32_t>(min(static_cast<long long>(tile), doc_count - first));
    const float* row = scores + static_cast<std::size_t>(q) * doc_count + first;
    std::uint64_t lo = ~0ull;
    std::uint64_t hi = 0ull;
    gatherRounds(n, [&](std::uint32_t i) { return makeKey(row[i], static_cast<std::uint32_t>(first + i)); },
                 [&](std::uint32_t i, std::uint64_t key) {
                     lds_keys[i] = key;
                     lo = min(lo, key);
                     hi = max(hi, key);
                 });
    if (t == 0) {
        lds.count = 0u;
    }
    // (ldsSelectCut's first barrier also makes the keys and the count visible)
    const std::uint64_t cut = ldsSelectCut(lds_keys, n, k, lo, hi, lds);
    ldsCollect(lds_keys, n, cut, out, static_cast<std::uint32_t>(k), lds);  // exactly min(n, k) keys
    __syncthreads();
    const std::uint32_t taken = min(lds.count, static_cast<std::uint32_t>(k));
    for (std::uint32_t i = taken + static_cast<std::uint32_t>(t); i < static_cast<std::uint32_t>(k); i += blockDim.x) {
        out[i] = 0ull;
    }
}

// ---- candidate merge (one block per query, merge.hpp) -------------------------------------------

__global__ __launch_bounds__(kMergeThreads) void selectMergeKernel(
    MergeInputs in, int k, int batch, std::uint64_t* __restrict__ out_keys,
    std::uint64_t* __restrict__ threshold, std::uint32_t* __restrict__ overflow,
    int* __restrict__ out_index, float* __restrict__ out_score) {
    __shared__ MergeLds lds;
    mergeQuery(in, k, batch, out_keys, threshold, overflow, out_index, out_score, static_cast<int>(blockIdx.x), lds);
}

// ---- merge of sorted segments (one block per query) ---------------------------------------------

constexpr int kSortedMergeThreads = 256;

// Every segment s holds c_s <= k keys in descending order. With T the k-th largest non-zero
// segment head (or every key when fewer than k heads are non-zero), the k best keys are all at
// least T (k heads are), and each lies in a segment whose head is at least T: at most k segments
// of at most k keys, ranked by comparison.
__global__ __launch_bounds__(kSortedMergeThreads) void sortedSegmentMergeKernel(
    MergeInputs in, int k, int batch, std::uint64_t* __restrict__ out_keys, std::uint32_t* __restrict__ overflow,
    int* __restrict__ out_index, float* __restrict__ out_score) {
    __shared__ std::uint64_t lds_head[kSortedMergeMaxSegments];
    __shared__ std::uint32_t lds_count[kSortedMergeMaxSegments];
    __shared__ int lds_segs[kSortedMergeMaxK];
    __shared__ std::uint64_t lds_pick[kSortedMergeMaxK * kSortedMergeMaxK];
    __shared__ std::uint64_t lds_cut;
    __shared__ std::uint32_t lds_nsegs;
    __shared__ std::uint32_t lds_taken;

    const int q = blockIdx.x;
    const int t = threadIdx.x;
    const int n_seg = in.n_seg;
    const std::uint32_t cap = 1u << in.seg_log2;
    auto segment = [&](int s) { return in.seg + ((static_cast<std::size_t>(s) * batch + q) << in.seg_log2); };
    for (int s = t; s < n_seg; s += kSortedMergeThreads) {
        // both loads at once: the first slot is read whatever the count (an empty segment's slot
        // holds a stale key, which the count then discards)
        const std::uint32_t c = min(in.seg_count[static_cast<std::size_t>(s) * batch + q], cap);
        const std::uint64_t first = segment(s)[0];
        lds_count[s] = c;
        lds_head[s] = c > 0u ? first : 0ull;
    }
    if (t == 0) {
        lds_cut = 1ull;  // fewer than k non-zero heads: every non-zero key
        lds_nsegs = 0u;
        lds_taken = 0u;
    }
    __syncthreads();
    for (int s = t; s < n_seg; s += kSortedMergeThreads) {
        const std::uint64_t head = lds_head[s];
        if (head != 0ull) {
            int above = 0;
            for (int j = 0; j < n_seg; ++j) {
                above += lds_head[j] > head ? 1 : 0;
            }
            if (above == k - 1) {
                lds_cut = head;
            }
        }
    }
    __syncthreads();
    const std::uint64_t cut = lds_cut;
    for (int s = t; s < n_seg; s += kSortedMergeThreads) {
        if (lds_head[s] >= cut) {  // (a zero head never reaches cut >= 1)
            lds_segs[atomicAdd(&lds_nsegs, 1u)] = s;  // at most k segments
        }
    }
    __syncthreads();
    const int nsegs = static_cast<int>(lds_nsegs);
    for (int i = t; i < nsegs * k; i += kSortedMergeThreads) {
        const int s = lds_segs[i / k];
        const int j = i - (i / k) * k;
        if (static_cast<std::uint32_t>(j) < lds_count[s]) {
            const std::uint64_t key = segment(s)[j];
            if (key >= cut) {
                lds_pick[atomicAdd(&lds_taken, 1u)] = key;  // at most k * k keys
            }
        }
    }
    __syncthreads();
    const int picked = static_cast<int>(lds_taken);
    const int taken = min(picked, k);
    std::uint64_t* dst = out_keys + static_cast<std::size_t>(q) * k;
    for (int i = t; i < picked; i += kSortedMergeThreads) {
        const std::uint64_t key = lds_pick[i];
        int rank = 0;
        for (int j = 0; j < picked; ++j) {
            rank += lds_pick[j] > key ? 1 : 0;  // keys are unique
        }
        if (rank < k) {
            dst[rank] = key;
            if (out_index != nullptr) {
                const std::size_t o = static_cast<std::size_t>(q) * k + rank;
                writeHit(key, &out_index[o], &out_score[o]);
            }
        }
    }
    for (int i = taken + t; i < k; i += kSortedMergeThreads) {
        dst[i] = 0ull;
        if (out_index != nullptr) {
            const std::size_t o = static_cast<std::size_t>(q) * k + i;
            writeHit(0ull, &out_index[o], &out_score[o]);
        }
    }
    if (t == 0 && overflow != nullptr && in.reset_overflow) {
        overflow[q] = 0u;  // (no segment holds more than its k keys)
    }
}

// The same selection for kSortedMergeMaxK < k <= kSortedSelectMaxK: the keys >= the k-th best head
// in the segments whose head reaches it (at most k segments of at most k keys, so at most
// kSelectLdsKeys keys) go to LDS, the best k of them are found by radix passes (ldsSelectCut) and
// only those k are ranked by comparison.
__global__ __launch_bounds__(kMergeThreads) void sortedSegmentSelectKernel(
    MergeInputs in, int k, int batch, std::uint64_t* __restrict__ out_keys, std::uint32_t* __restrict__ overflow,
    int* __restrict__ out_index, float* __restrict__ out_score) {
    __shared__ std::uint64_t lds_head[kSortedMergeMaxSegments];
    __shared__ std::uint32_t lds_count[kSortedMergeMaxSegments];
    __shared__ int lds_segs[kSortedSelectMaxK];
    __shared__ std::uint64_t lds_pick[kSortedSelectMaxK * kSortedSelectMaxK];
    __shared__ std::uint64_t lds_top[kSortedSelectMaxK];
    __shared__ LdsSelect lds;
    __shared__ std::uint64_t lds_cut;
    __shared__ std::uint32_t lds_nsegs;
    __shared__ std::uint32_t lds_picked;

    const int q = blockIdx.x;
    const int t = threadIdx.x;
    const int n_seg = in.n_seg;
    // a segment holds at most k keys (the scan writes min(count, k)); the clamp keeps the picks
    // within k * k whatever the counts say
    const std::uint32_t cap = min(1u << in.seg_log2, static_cast<std::uint32_t>(k));
    auto segment = [&](int s) { return in.seg + ((static_cast<std::size_t>(s) * batch + q) << in.seg_log2); };
    for (int s = t; s < n_seg; s += blockDim.x) {
        const std::uint32_t c = min(in.seg_count[static_cast<std::size_t>(s) * batch + q], cap);
        const std::uint64_t first = segment(s)[0];
        lds_count[s] = c;
        lds_head[s] = c > 0u ? first : 0ull;
    }
    if (t == 0) {
        lds_cut = 1ull;  // fewer than k non-zero heads: every non-zero key
        lds_nsegs = 0u;
        lds_picked = 0u;
        lds.count = 0u;
    }
    __syncthreads();
    for (int s = t; s < n_seg; s += blockDim.x) {
        const std::uint64_t head = lds_head[s];
        if (head != 0ull) {
            int above = 0;
            for (int j = 0; j < n_seg; ++j) {
                above += lds_head[j] > head ? 1 : 0;
            }
            if (above == k - 1) {
                lds_cut = head;
            }
        }
    }
    __syncthreads();
    const std::uint64_t cut = lds_cut;
    for (int s = t; s < n_seg; s += blockDim.x) {
        if (lds_head[s] >= cut) {  // (a zero head never reaches cut >= 1)
            lds_segs[atomicAdd(&lds_nsegs, 1u)] = s;  // at most k segments
        }
    }
    __syncthreads();
    const std::uint32_t slots = lds_nsegs * static_cast<std::uint32_t>(k);
    std::uint64_t lo = ~0ull;
    std::uint64_t hi = 0ull;
    // slot i: key i % k of chosen segment i / k (0 past the segment's count); each thread's loads
    // of a round are in flight together
    gatherRounds(slots,
                 [&](std::uint32_t i) {
                     const int s = lds_segs[i / k];
                     const std::uint32_t j = i - (i / k) * k;
                     return j < lds_count[s] ? segment(s)[j] : 0ull;
                 },
                 [&](std::uint32_t, std::uint64_t key) {
                     if (key != 0ull && key >= cut) {
                         lds_pick[atomicAdd(&lds_picked, 1u)] = key;  // at most k * k keys
                         lo = min(lo, key);
                         hi = max(hi, key);
                     }
                 });
    __syncthreads();  // every pick and their count
    const std::uint32_t n = lds_picked;
    const std::uint64_t top_cut = ldsSelectCut(lds_pick, n, k, lo, hi, lds);
    ldsCollect(lds_pick, n, top_cut, lds_top, static_cast<std::uint32_t>(k), lds);  // exactly min(n, k)
    __syncthreads();
    const int taken = static_cast<int>(min(lds.count, static_cast<std::uint32_t>(k)));
    std::uint64_t* dst = out_keys + static_cast<std::size_t>(q) * k;
    for (int i = t; i < taken; i += blockDim.x) {
        const std::uint64_t key = lds_top[i];
        int rank = 0;
        for (int j = 0; j < taken; ++j) {
            rank += lds_top[j] > key ? 1 : 0;  // keys are unique
        }
        dst[rank] = key;
        if (out_index != nullptr) {
            const std::size_t o = static_cast<std::size_t>(q) * k + rank;
            writeHit(key, &out_index[o], &out_score[o]);
        }
    }
    for (int i = taken + t; i < k; i += blockDim.x) {
        dst[i] = 0ull;
        if (out_index != nullptr) {
            const std::size_t o = static_cast<std::size_t>(q) * k + i;
            writeHit(0ull, &out_index[o], &out_score[o]);
        }
    }
    if (t == 0 && overflow != nullptr && in.reset_overflow) {
        overflow[q] = 0u;  // (no segment holds more than its k keys)
    }
}

// ---- thresholds from a sketch phase (one block per query) ----------------------------------------

constexpr int kSketchThreads = 256;
constexpr int kSketchPerThread = kMaxSketchSlots / kSketchThreads;  // slot scores per thread
constexpr int kSketchBins = 2048;                                    // 11-bit digits
constexpr int kSketchBinsPerThread = kSketchBins / kSketchThreads;

// The j-th and k-th best of a query's slot scores: a radix select over the scores' ordered bits in
// three passes (digits of bits 31..21, 20..10 and 9..0), both ranks in the same passes. A pass
// counts, per rank, the scores whose higher digits equal that rank's prefix so far into an LDS
// histogram (rank j's count in the low 16 bits of a bin, rank k's in the high 16 bits; at most
// 2048 scores, so neither half carries), then a block scan over the bins in descending digit order
// finds the bin that holds the rank, which fixes the digit and the rank left within the bin.
__global__ __launch_bounds__(kSketchThreads) void sketchThresholdKernel(const float* __restrict__ sketch, int slots,
                                                                        int batch, int j, int k,
                                                                        std::uint64_t* __restrict__ tau,
                                                                        std::uint64_t* __restrict__ tau_safe,
                                                                        std::uint32_t* __restrict__ flag_count) {
    __shared__ std::uint32_t hist[kSketchBins];
    __shared__ std::uint32_t wave_sums[kSketchThreads / kWave];
    __shared__ std::uint32_t pick[2][2];  // per rank: the digit, the scores in higher bins
    const int q = blockIdx.x;
    const int t = threadIdx.x;
    // the slot scores' ordered bits; an empty slot (-inf: it saw no row) and the padding are 0
    std::uint32_t v[kSketchPerThread];
#pragma unroll
    for (int r = 0; r < kSketchPerThread; ++r) {
        const int s = r * kSketchThreads + t;
        const float x = s < slots ? sketch[static_cast<std::size_t>(s) * batch + q] : -INFINITY;
        v[r] = x > -INFINITY ? orderedBits(x) : 0u;
    }
    if (q == 0 && t == 0) {
        *flag_count = 0u;
    }
    std::uint32_t prefix[2] = {0u, 0u};
    std::uint32_t rank[2] = {static_cast<std::uint32_t>(j), static_cast<std::uint32_t>(k)};
    constexpr int kShift[3] = {21, 10, 0};
    constexpr int kBits[3] = {11, 11, 10};
#pragma unroll
    for (int p = 0; p < 3; ++p) {
        const int shift = kShift[p];
        const int high = shift + kBits[p];  // the digits above this one start here (32: none)
        const std::uint32_t digit_mask = (1u << kBits[p]) - 1u;
#pragma unroll
        for (int b = 0; b < kSketchBinsPerThread; ++b) {
            hist[b * kSketchThreads + t] = 0u;
        }
        __syncthreads();
        // a score matches both ranks' prefixes only when they are equal, so one add per score
#pragma unroll
        for (int r = 0; r < kSketchPerThread; ++r) {
            const std::uint32_t upper = high < 32 ? v[r] >> (high & 31) : 0u;
            const std::uint32_t add = (upper == (high < 32 ? prefix[0] >> (high & 31) : 0u) ? 1u : 0u) +
                                      (upper == (high < 32 ? prefix[1] >> (high & 31) : 0u) ? 0x10000u : 0u);
            if (add != 0u) {
                atomicAdd(&hist[(v[r] >> shift) & digit_mask], add);
            }
        }
        __syncthreads();
        // thread t takes the bins kSketchBins - 1 - 8t - b (b < 8): all bins in descending order
        std::uint32_t own[kSketchBinsPerThread];
        std::uint32_t sum = 0u;
#pragma unroll
        for (int b = 0; b < kSketchBinsPerThread; ++b) {
            own[b] = hist[kSketchBins - 1 - kSketchBinsPerThread * t - b];
            sum += own[b];
        }
        std::uint32_t total;
        std::uint32_t running = blockInclusiveSum<kSketchThreads>(sum, wave_sums, &total) - sum;
#pragma unroll
        for (int b = 0; b < kSketchBinsPerThread; ++b) {
            const std::uint32_t next = running + own[b];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const std::uint32_t above = (running >> (16 * i)) & 0xFFFFu;
                const std::uint32_t through = (next >> (16 * i)) & 0xFFFFu;
                if (above < rank[i] && through >= rank[i]) {
                    pick[i][0] = static_cast<std::uint32_t>(kSketchBins - 1 - kSketchBinsPerThread * t - b);
                    pick[i][1] = above;
                }
            }
            running = next;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            prefix[i] |= pick[i][0] << shift;
            rank[i] -= pick[i][1];
        }
    }
    // every score >= the j-th (k-th) best slot score; 0 when that slot is empty or missing
    if (t == 0) {
        tau[q] = j <= slots ? static_cast<std::uint64_t>(prefix[0]) << 32 : 0ull;
        tau_safe[q] = k <= slots ? static_cast<std::uint64_t>(prefix[1]) << 32 : 0ull;
    }
}

int topkScratchElements(int doc_count, int k) {
    if (doc_count <= 0 || k <= 0) {
        return 0;
    }
    const long long reference = static_cast<long long>((doc_count + kTileSize - 1) / kTileSize) * k;
    const long long needed = std::max<long long>(kMinScratchElements, 2LL * k + 16);
    return static_cast<int>(std::max(reference, needed));
}

}  // namespace

int launchSelectMerge(const MergeInputs& in, int k, int batch, std::uint64_t* out_keys,
                      std::uint64_t* threshold, std::uint32_t* overflow, int* out_index,
                      float* out_score, hipStream_t stream) {
    if (in.n_seg > kMaxSegments) {
        return setError(ZCGVS_ERR_RUNTIME, "zcgvs select: too many candidate segments");
    }
    selectMergeKernel<<<batch, kMergeThreads, 0, stream>>>(in, k, batch, out_keys, threshold,
                                                            overflow, out_index, out_score);
    ZCGVS_LAUNCH_CHECK("select merge");
    return ZCGVS_OK;
}

int launchSketchThreshold(const float* sketch, int slots, int batch, int j, int k, std::uint64_t* tau,
                          std::uint64_t* tau_safe, std::uint32_t* flag_count, hipStream_t stream) {
    if (slots < 1 || slots > kMaxSketchSlots || j < 1 || k < 1) {
        return setError(ZCGVS_ERR_RUNTIME, "zcgvs select: sketch threshold shape out of range");
    }
    sketchThresholdKernel<<<batch, kSketchThreads, 0, stream>>>(sketch, slots, batch, j, k, tau, tau_safe,
                                                                  flag_count);
    ZCGVS_LAUNCH_CHECK("sketch threshold");
    return ZCGVS_OK;
}

int launchSortedSegmentMerge(const MergeInputs& in, int k, int batch, std::uint64_t* out_keys,
                             std::uint32_t* overflow, int* out_index, float* out_score, hipStream_t stream) {
    if (k > kSortedMergeMaxK && k <= kSortedSelectMaxK && in.n_seg >= 1 && in.n_seg <= kSortedMergeMaxSegments &&
        in.seg != nullptr && in.prev == nullptr && in.dense == nullptr && (1 << in.seg_log2) >= k) {
        sortedSegmentSelectKernel<<<batch, kMergeThreads, 0, stream>>>(in, k, batch, out_keys, overflow, out_index,
                                                                       out_score);
        ZCGVS_LAUNCH_CHECK("sorted-segment select");
        return ZCGVS_OK;
    }
    if (k < 1 || k > kSortedMergeMaxK || in.n_seg < 1 || in.n_seg > kSortedMergeMaxSegments || in.seg == nullptr ||
        in.prev != nullptr || in.dense != nullptr || (1 << in.seg_log2) < k) {
        return setError(ZCGVS_ERR_RUNTIME, "zcgvs select: sorted-segment merge does not take this shape");
    }
    sortedSegmentMergeKernel<<<batch, kSortedMergeThreads, 0, stream>>>(in, k, batch, out_keys, overflow,
                                                                        out_index, out_score);
    ZCGVS_LAUNCH_CHECK("sorted-segment merge");
    return ZCGVS_OK;
}

}  // namespace zcgvs_hip

using namespace zcgvs_hip;

extern "C" {

int zcgvs_topk_tile_size(void) { return kTileSize; }
int zcgvs_topk_merge_tile(void) { return kMergeTile; }
int zcgvs_topk_max_k(void) { return kMaxK; }

int zcgvs_topk_block_count(int doc_count) {
    if (doc_count <= 0) {
        return 0;
    }
    return (doc_count + kTileSize - 1) / kTileSize;
}

int zcgvs_topk_scratch_elements(int doc_count, int k) { return topkScratchElements(doc_count, k); }

int zcgvs_launch_topk(const float* d_scores, int doc_count, int k, int batch, int* d_out_indices,
                      float* d_out_values, float* d_scratch_values_a, int* d_scratch_indices_a,
                      float* d_scratch_values_b, int* d_scratch_indices_b,
                      zcgvs_stream_t stream) {
    (void)d_scratch_values_b;
    (void)d_scratch_indices_b;
    if (k <= 0 || doc_count <= 0 || batch <= 0) {
        return clearError();
    }
    if (k > kMaxK) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT,
                        "zcgvs top-k: k=" + std::to_string(k) + " exceeds per-tile capacity " +
                            std::to_string(kMaxK));
    }
    if (k > doc_count) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT,
                        "zcgvs top-k: k=" + std::to_string(k) + " exceeds candidate count " +
                            std::to_string(doc_count));
    }
    if (d_scores == nullptr || d_out_indices == nullptr || d_out_values == nullptr ||
        d_scratch_values_a == nullptr || d_scratch_indices_a == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs top-k: null device pointer");
    }
    // Every tile's best k keys (topkTileKernel), then the per-query merge of the tile winners
    // (merge.hpp), which writes the result in (score desc, index asc) order. When the winners of a
    // query exceed the merge's LDS gather, groups of tiles are merged first, each (query, group)
    // pair as a merge query of its own, and the group results after. Scratch b holds the winners,
    // scratch a the group results or the final keys, scratch values b the final keys after
    // groups; all fit the per-query size of topkScratchElements (at least 2k + 16 words and
    // ceil(N / 1024) * k, against 2 * ceil(N / 8192) * k words of winners and 2 * 12 * k of groups).
    const std::size_t elements = static_cast<std::size_t>(topkScratchElements(doc_count, k)) & ~std::size_t(1);
    const long long tile = topkTileScores(doc_count, k);
    const long long tiles = (doc_count + tile - 1) / tile;
    const long long lds_keys = static_cast<long long>(kSelectLdsKeys);
    const bool grouped = tiles * k > lds_keys;
    // groups of tiles_per_group tiles (the last ones padded with empty tiles)
    const long long groups = grouped ? std::min<long long>(tiles, std::max<long long>(2, lds_keys / k)) : 1;
    const long long tiles_per_group = (tiles + groups - 1) / groups;
    const long long padded = groups * tiles_per_group;
    const std::size_t stride = static_cast<std::size_t>(padded) * static_cast<std::size_t>(k);  // winner keys per query
    if (stride > elements / 2 || static_cast<std::size_t>(groups) * k > elements / 2 || padded > INT32_MAX ||
        (grouped && (d_scratch_values_b == nullptr || 2 * static_cast<std::size_t>(k) > elements))) {
        return setError(ZCGVS_ERR_RUNTIME, "zcgvs top-k: tile winners exceed the scratch");
    }
    std::uint64_t* winners = reinterpret_cast<std::uint64_t*>(d_scratch_indices_a);
    const hipStream_t s = toStream(stream);
    topkTileKernel<<<dim3(static_cast<unsigned>(padded), static_cast<unsigned>(batch)), kMergeThreads, 0, s>>>(
        d_scores, doc_count, static_cast<int>(tile), k, winners, stride);
    ZCGVS_LAUNCH_CHECK("top-k tiles");
    MergeInputs in;
    in.dense = winners;
    in.n_dense = tiles_per_group * k;
    in.dense_stride = tiles_per_group * k;  // merge query q * groups + g: group g of query q
    std::uint64_t* keys = reinterpret_cast<std::uint64_t*>(d_scratch_values_a);
    if (grouped) {
        const int status = launchSelectMerge(in, k, batch * static_cast<int>(groups), keys, nullptr, nullptr,
                                             nullptr, nullptr, s);
        if (status != ZCGVS_OK) {
            return status;
        }
        in = MergeInputs{};
        in.dense = keys;
        in.n_dense = groups * k;
        in.dense_stride = groups * k;
        keys = reinterpret_cast<std::uint64_t*>(d_scratch_values_b);
    }
    const int status = launchSelectMerge(in, k, batch, keys, nullptr, nullptr, d_out_indices, d_out_values, s);
    if (status != ZCGVS_OK) {
        return status;
    }
    return clearError();
}

}  // extern "C"
