// The per-query candidate merge of the fused search: one 1024-thread block selects a query's
// best k keys from the keys kept by earlier phases, a dense phase's fixed slots and the
// per-workgroup candidate segments of a threshold phase (MergeInputs), by exact radix passes over
// the unique 64-bit keys. topk.hip launches it on its own; recover.hip fuses it with the exact
// fallback of the query it flags.
#pragma once

#include "common.hpp"
#include "select.hpp"

namespace zcgvs_hip {

namespace {

constexpr int kMaxSegments = 4096;

// Applies f to every non-zero key of query q's candidate set (see MergeInputs).
template <typename F>
__device__ __forceinline__ void forEachCandidate(const MergeInputs& in, int q, int batch,
                                                 const std::uint32_t* seg_valid, F&& f) {
    if (in.prev != nullptr) {
        const std::uint64_t* prev = in.prev + static_cast<std::size_t>(q) * in.k_prev;
        for (int i = threadIdx.x; i < in.k_prev; i += blockDim.x) {
            const std::uint64_t key = prev[i];
            if (key != 0ull) {
                f(key);
            }
        }
    }
    if (in.dense != nullptr) {
        const std::uint64_t* dense = in.dense + static_cast<std::size_t>(q) * in.dense_stride;
#pragma unroll 8
        for (long long i = threadIdx.x; i < in.n_dense; i += blockDim.x) {
            const std::uint64_t key = dense[i];
            if (key != 0ull) {
                f(key);
            }
        }
    }
    if (in.seg != nullptr) {
        const long long total = static_cast<long long>(in.n_seg) << in.seg_log2;
        const long long mask = (1LL << in.seg_log2) - 1;
#pragma unroll 8
        for (long long i = threadIdx.x; i < total; i += blockDim.x) {
            const int s = static_cast<int>(i >> in.seg_log2);
            const long long j = i & mask;
            if (j < static_cast<long long>(seg_valid[s])) {
                const std::uint64_t key =
                    in.seg[((static_cast<std::size_t>(s) * batch + q) << in.seg_log2) + j];
                if (key != 0ull) {
                    f(key);
                }
            }
        }
    }
}

// Candidate sets of up to kSelectLdsKeys keys are first gathered into LDS, so the radix passes
// read LDS instead of re-walking the segments in global memory; larger sets take the same
// passes over global memory. The gather needs no load results to place a key: previous keys
// and dense keys are copied as they lie (zero keys are skipped later), and segment j of
// segment s goes to offset[s] + j, from the exclusive scan of the segment counts.
constexpr std::uint32_t kSelectLdsKeys = 12288;
static_assert(kMaxK <= kSelectBins, "the ranks of a selection reuse the histogram");

// Visits elements 0..n-1 (n uniform) with the block's threads, kBatch per thread per round:
// `load(i)` for each of a thread's elements of the round first (an index past n is clamped to
// n - 1, so every load reads inside the source), then `use(i, value)` for those below n.
// Keeping the loads of a round apart from their uses lets them all be in flight at once.
template <int kBatch, typename Load, typename Use>
__device__ __forceinline__ void gatherRoundsOf(std::uint32_t n, Load& load, Use& use) {
    const std::uint32_t t = threadIdx.x;
    for (std::uint32_t r0 = 0; r0 < n; r0 += kBatch * blockDim.x) {
        std::uint64_t value[kBatch];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            value[b] = load(min(r0 + b * blockDim.x + t, n - 1u));
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const std::uint32_t i = r0 + b * blockDim.x + t;
            if (i < n) {
                use(i, value[b]);
            }
        }
    }
}

// The batch is the smallest of 1, 2, 4 or 8 that covers n in one round (8 beyond), so no thread
// loads more clamped duplicates than needed.
template <typename Load, typename Use>
__device__ __forceinline__ void gatherRounds(std::uint32_t n, Load&& load, Use&& use) {
    const std::uint32_t threads = blockDim.x;
    if (n <= threads) {
        gatherRoundsOf<1>(n, load, use);
    } else if (n <= 2u * threads) {
        gatherRoundsOf<2>(n, load, use);
    } else if (n <= 4u * threads) {
        gatherRoundsOf<4>(n, load, use);
    } else {
        gatherRoundsOf<8>(n, load, use);
    }
}

// LDS of one query's merge (a struct, so a kernel that runs more after the merge can reuse it).
struct MergeLds {
    std::uint32_t hist[kSelectBins];
    std::uint32_t scan[kMergeThreads / kWave];
    std::uint64_t keys[kMaxK];
    std::uint32_t seg[kMaxSegments];     // valid count per segment
    std::uint32_t offset[kMaxSegments];  // exclusive scan of seg
    std::uint64_t cand[kSelectLdsKeys];
    SelectState state;
    std::uint32_t valid;
    std::uint32_t overflow;
    std::uint32_t flagged;
    std::uint32_t wave_count[kMergeThreads / kWave];
    std::uint64_t wave_lo[kMergeThreads / kWave];
    std::uint64_t wave_hi[kMergeThreads / kWave];
    std::uint64_t kth;  // the k-th best key (0: fewer than k keys)
};

// The merge of query q by the whole block (kMergeThreads threads), see MergeInputs. Returns,
// uniformly over the block, whether a final merge flagged the query for the exact fallback; the
// block's LDS use is over when it returns.
__device__ __forceinline__ bool mergeQuery(const MergeInputs& in, int k, int batch, std::uint64_t* __restrict__ out_keys,
                                           std::uint64_t* __restrict__ threshold, std::uint32_t* __restrict__ overflow,
                                           int* __restrict__ out_index, float* __restrict__ out_score, int q,
                                           MergeLds& lds) {
    std::uint32_t(&lds_hist)[kSelectBins] = lds.hist;
    std::uint32_t(&lds_scan)[kMergeThreads / kWave] = lds.scan;
    std::uint64_t(&lds_keys)[kMaxK] = lds.keys;
    std::uint32_t(&lds_seg)[kMaxSegments] = lds.seg;
    std::uint32_t(&lds_offset)[kMaxSegments] = lds.offset;
    std::uint64_t(&lds_cand)[kSelectLdsKeys] = lds.cand;
    SelectState& lds_state = lds.state;
    std::uint32_t& lds_valid = lds.valid;
    std::uint32_t& lds_overflow = lds.overflow;
    std::uint32_t(&lds_wave_count)[kMergeThreads / kWave] = lds.wave_count;
    std::uint64_t(&lds_wave_lo)[kMergeThreads / kWave] = lds.wave_lo;
    std::uint64_t(&lds_wave_hi)[kMergeThreads / kWave] = lds.wave_hi;
    std::uint64_t& lds_kth = lds.kth;

    const int t = threadIdx.x;
    if (t == 0) {
        lds_kth = 0ull;
        lds.flagged = 0u;
        if (in.zero_count != nullptr && q == 0) {
            *in.zero_count = 0u;
        }
        lds_valid = 0u;
        lds_overflow = 0u;
        lds_state.prefix = 0ull;
        lds_state.bits = 0u;
        lds_state.need = static_cast<std::uint32_t>(k);
        lds_state.count = 0u;
    }
    __syncthreads();
    const std::uint32_t k_prev = in.prev != nullptr ? static_cast<std::uint32_t>(in.k_prev) : 0u;
    const std::uint32_t n_dense = in.dense != nullptr ? static_cast<std::uint32_t>(in.n_dense) : 0u;
    // Count, smallest and largest non-zero key of what this thread gathers (then reduced over
    // the block), so the radix passes can start below the bits every key shares.
    std::uint32_t own_count = 0u;
    std::uint64_t own_lo = ~0ull;
    std::uint64_t own_hi = 0ull;
    auto note = [&](std::uint64_t key) {
        if (key != 0ull) {
            ++own_count;
            own_lo = min(own_lo, key);
            own_hi = max(own_hi, key);
        }
    };
    std::uint32_t seg_total = 0u;
    if (in.n_seg > 0) {  // (uniform: a kernel argument)
        const std::uint32_t cap = 1u << in.seg_log2;
        for (int s = t; s < in.n_seg; s += blockDim.x) {
            const std::uint32_t c = in.seg_count[static_cast<std::size_t>(s) * batch + q];
            lds_seg[s] = min(c, cap);
            if (c > cap) {
                lds_overflow = 1u;
            }
        }
        __syncthreads();
        // Exclusive scan of the segment counts: thread t owns a contiguous run of segments.
        const int per_thread = (in.n_seg + kMergeThreads - 1) / kMergeThreads;
        std::uint32_t run = 0u;
        for (int i = 0; i < per_thread; ++i) {
            const int s = t * per_thread + i;
            run += s < in.n_seg ? lds_seg[s] : 0u;
        }
        std::uint32_t acc = blockInclusiveSum<kMergeThreads>(run, lds_scan, &seg_total) - run;
        for (int i = 0; i < per_thread; ++i) {
            const int s = t * per_thread + i;
            if (s < in.n_seg) {
                lds_offset[s] = acc;
                acc += lds_seg[s];
            }
        }
    }
    const std::uint64_t gathered = static_cast<std::uint64_t>(k_prev) + n_dense + seg_total;
    const bool in_lds = gathered <= kSelectLdsKeys;
    __syncthreads();

    if (in_lds) {
        // Each thread handles up to eight keys at a time: their sources are found first (a
        // segment search in LDS for segment keys) and all their loads are issued before any
        // result is used, so the loads of one round are in flight together.
        if (k_prev > 0u) {
            const std::uint64_t* prev = in.prev + static_cast<std::size_t>(q) * in.k_prev;
            gatherRounds(k_prev, [&](std::uint32_t i) { return prev[i]; },
                         [&](std::uint32_t i, std::uint64_t key) {
                             lds_cand[i] = key;
                             note(key);
                         });
        }
        if (n_dense > 0u) {
            const std::uint64_t* dense = in.dense + static_cast<std::size_t>(q) * in.dense_stride;
            gatherRounds(n_dense, [&](std::uint32_t i) { return dense[i]; },
                         [&](std::uint32_t i, std::uint64_t key) {
                             lds_cand[k_prev + i] = key;
                             note(key);
                         });
        }
        if (in.seg != nullptr && seg_total > 0u) {
            // Candidate i of the compacted list lives in the last segment whose offset is
            // <= i (empty segments share their successor's offset), at position i - offset.
            // The search takes ceil(log2(n_seg)) halving steps for every key (a step after
            // convergence keeps the segment), so the steps of a thread's keys run side by side.
            const std::uint32_t base = k_prev + n_dense;
            const int steps = in.n_seg > 1 ? 32 - __clz(static_cast<std::uint32_t>(in.n_seg - 1)) : 0;
            gatherRounds(seg_total,
                         [&](std::uint32_t i) {
                             int lo = 0;
                             int hi = in.n_seg - 1;
                             for (int step = 0; step < steps; ++step) {
                                 const int mid = (lo + hi + 1) >> 1;
                                 if (lds_offset[mid] <= i) {
                                     lo = mid;
                                 } else {
                                     hi = mid - 1;
                                 }
                             }
                             const std::uint32_t j = i - lds_offset[lo];
                             return in.seg[((static_cast<std::size_t>(lo) * batch + q) << in.seg_log2) + j];
                         },
                         [&](std::uint32_t i, std::uint64_t key) {
                             lds_cand[base + i] = key;
                             note(key);
                         });
        }
    } else {
        forEachCandidate(in, q, batch, lds_seg, note);
    }

    auto forEachKey = [&](auto&& f) {
        if (in_lds) {
            const std::uint32_t n = static_cast<std::uint32_t>(gathered);
            for (std::uint32_t i = t; i < n; i += blockDim.x) {
                const std::uint64_t key = lds_cand[i];
                if (key != 0ull) {
                    f(key);
                }
            }
        } else {
            forEachCandidate(in, q, batch, lds_seg, f);
        }
    };

    // Count, smallest and largest valid key: wavefront reductions, one LDS slot per wavefront,
    // then wavefront 0 reduces the slots (a block-wide atomic on one word would serialize 1024
    // updates).
    {
        const std::uint64_t count = waveReduce64(own_count, [](std::uint64_t a, std::uint64_t b) { return a + b; });
        const std::uint64_t lo = waveReduce64(own_lo, [](std::uint64_t a, std::uint64_t b) { return min(a, b); });
        const std::uint64_t hi = waveReduce64(own_hi, [](std::uint64_t a, std::uint64_t b) { return max(a, b); });
        if ((t & (kWave - 1)) == 0) {
            lds_wave_count[t / kWave] = static_cast<std::uint32_t>(count);
            lds_wave_lo[t / kWave] = lo;
            lds_wave_hi[t / kWave] = hi;
        }
    }
    __syncthreads();  // (also: the gathered keys are in LDS)
    if (t < kWave) {
        constexpr int kSlots = kMergeThreads / kWave;
        std::uint64_t count = t < kSlots ? lds_wave_count[t] : 0ull;
        std::uint64_t lo = t < kSlots ? lds_wave_lo[t] : ~0ull;
        std::uint64_t hi = t < kSlots ? lds_wave_hi[t] : 0ull;
        count = waveReduce64(count, [](std::uint64_t a, std::uint64_t b) { return a + b; });
        lo = waveReduce64(lo, [](std::uint64_t a, std::uint64_t b) { return min(a, b); });
        hi = waveReduce64(hi, [](std::uint64_t a, std::uint64_t b) { return max(a, b); });
        if (t == 0) {
            lds_valid = static_cast<std::uint32_t>(count);
            lds_state.done = count <= static_cast<std::uint64_t>(k) ? 1u : 0u;
            if (count > static_cast<std::uint64_t>(k)) {
                // The keys (unique, at least two) share their top `common` bits: the radix
                // passes start below them, so the first digit already separates the keys.
                const int common = __clzll(hi ^ lo);
                lds_state.prefix = common == 0 ? 0ull : (hi >> (64 - common));
                lds_state.bits = static_cast<std::uint32_t>(common);
            }
        }
    }
    __syncthreads();
    const std::uint32_t n_valid = lds_valid;

    for (int pass = 0; pass < kSelectPasses && !lds_state.done; ++pass) {
        const int width = min(11, 64 - static_cast<int>(lds_state.bits));
        for (int i = t; i < (1 << width); i += blockDim.x) {
            lds_hist[i] = 0u;
        }
        __syncthreads();
        const std::uint32_t bits = lds_state.bits;
        const std::uint64_t prefix = lds_state.prefix;
        const int shift = 64 - static_cast<int>(bits) - width;
        const std::uint64_t digit_mask = (1ull << width) - 1ull;
        forEachKey([&](std::uint64_t key) {
            if (bits == 0u || (key >> (64 - bits)) == prefix) {
                atomicAdd(&lds_hist[(key >> shift) & digit_mask], 1u);
            }
        });
        __syncthreads();
        selectPickBucket<kMergeThreads>(lds_hist, width, &lds_state, lds_scan);
    }

    const std::uint64_t cut = n_valid <= static_cast<std::uint32_t>(k) ? 1ull : selectThreshold(lds_state);
    if (in_lds) {
        // one slot reservation per wavefront step (ballot, popcount, prefix count)
        const std::uint32_t n = static_cast<std::uint32_t>(gathered);
        for (std::uint32_t base = 0; base < n; base += blockDim.x) {
            const std::uint32_t i = base + static_cast<std::uint32_t>(t);
            const std::uint64_t key = i < n ? lds_cand[i] : 0ull;
            const bool take = key != 0ull && key >= cut;
            const std::uint64_t mask = __builtin_amdgcn_ballot_w64(take);
            if (mask != 0ull) {
                std::uint32_t first = 0u;
                if ((t & (kWave - 1)) == 0) {
                    first = atomicAdd(&lds_state.count, static_cast<std::uint32_t>(__builtin_popcountll(mask)));
                }
                first = __builtin_amdgcn_readfirstlane(first);
                const std::uint32_t slot = first + __builtin_amdgcn_mbcnt_hi(static_cast<std::uint32_t>(mask >> 32),
                                                                             __builtin_amdgcn_mbcnt_lo(static_cast<std::uint32_t>(mask), 0u));
                if (take && slot < static_cast<std::uint32_t>(kMaxK)) {
                    lds_keys[slot] = key;
                }
            }
        }
    } else {
        forEachCandidate(in, q, batch, lds_seg, [&](std::uint64_t key) {
            if (key >= cut) {
                const std::uint32_t slot = atomicAdd(&lds_state.count, 1u);
                if (slot < static_cast<std::uint32_t>(kMaxK)) {
                    lds_keys[slot] = key;
                }
            }
        });
    }
    __syncthreads();
    // exactly min(n_valid, k) keys were collected (keys are unique)
    const std::uint32_t taken = min(min(lds_state.count, static_cast<std::uint32_t>(kMaxK)),
                                    static_cast<std::uint32_t>(k));
    std::uint64_t* dst = out_keys + static_cast<std::size_t>(q) * k;
    if (out_index != nullptr) {
        // The search's result: every key at its rank, the number of selected keys above it. The
        // comparisons of one key are split over `parts` threads whose counts meet in LDS (the
        // histogram, free after the passes), so a short list takes one round of comparisons.
        std::uint32_t* rank_of = lds_hist;
        for (std::uint32_t i = static_cast<std::uint32_t>(t); i < taken; i += blockDim.x) {
            rank_of[i] = 0u;
        }
        __syncthreads();
        if (taken > 0u) {
            const std::uint32_t parts = max(1u, static_cast<std::uint32_t>(kMergeThreads) / taken);
            const std::uint32_t per = (taken + parts - 1u) / parts;
            for (std::uint32_t u = static_cast<std::uint32_t>(t); u < taken * parts; u += blockDim.x) {
                const std::uint32_t i = u / parts;
                const std::uint32_t j0 = (u - i * parts) * per;
                const std::uint32_t j1 = min(taken, j0 + per);
                const std::uint64_t key = lds_keys[i];
                std::uint32_t above = 0u;
                for (std::uint32_t j = j0; j < j1; ++j) {
                    above += lds_keys[j] > key ? 1u : 0u;
                }
                if (above != 0u) {
                    atomicAdd(&rank_of[i], above);
                }
            }
        }
        __syncthreads();
        for (std::uint32_t i = static_cast<std::uint32_t>(t); i < taken; i += blockDim.x) {
            const std::uint32_t rank = rank_of[i];
            const std::uint64_t key = lds_keys[i];
            dst[rank] = key;
            const std::size_t o = static_cast<std::size_t>(q) * k + rank;
            writeHit(key, &out_index[o], &out_score[o]);
            if (rank == static_cast<std::uint32_t>(k) - 1u) {
                lds_kth = key;
                if (threshold != nullptr) {
                    threshold[q] = key;
                }
            }
        }
    } else {
        // Between phases only the set and its smallest key (the threshold) matter: the keys stay
        // in collection order.
        std::uint64_t lo = ~0ull;
        for (std::uint32_t i = static_cast<std::uint32_t>(t); i < taken; i += blockDim.x) {
            const std::uint64_t key = lds_keys[i];
            dst[i] = key;
            lo = min(lo, key);
        }
        lo = waveReduce64(lo, [](std::uint64_t a, std::uint64_t b) { return min(a, b); });
        if ((t & (kWave - 1)) == 0) {
            lds_wave_lo[t / kWave] = lo;
        }
        __syncthreads();
        if (t < kWave) {  // wavefront 0 reduces the per-wavefront minima
            std::uint64_t v = t < kMergeThreads / kWave ? lds_wave_lo[t] : ~0ull;
            v = waveReduce64(v, [](std::uint64_t a, std::uint64_t b) { return min(a, b); });
            if (t == 0 && taken >= static_cast<std::uint32_t>(k)) {
                lds_kth = v;
                if (threshold != nullptr) {
                    threshold[q] = v;
                }
            }
        }
    }
    for (int i = static_cast<int>(taken) + t; i < k; i += blockDim.x) {
        dst[i] = 0ull;
        if (out_index != nullptr) {
            const std::size_t o = static_cast<std::size_t>(q) * k + i;
            writeHit(0ull, &out_index[o], &out_score[o]);
        }
    }
    __syncthreads();  // lds_kth and the threshold written above
    if (t == 0) {
        if (threshold != nullptr && taken < static_cast<std::uint32_t>(k)) {
            threshold[q] = 0ull;
        }
        if (in.final_merge) {
            const bool earlier = !in.reset_overflow && overflow[q] != 0u;
            const bool flagged = lds_overflow != 0u || earlier ||
                                 (in.require_full && taken < static_cast<std::uint32_t>(k));
            overflow[q] = flagged ? 1u : 0u;
            lds.flagged = flagged ? 1u : 0u;
            if (flagged) {
                const std::uint64_t kth = lds_kth;
                in.rerun_tau[q] = kth != 0ull ? kth - 1ull : (in.fallback_tau != nullptr ? in.fallback_tau[q] : 0ull);
                in.flag_list[atomicAdd(in.flag_count, 1u)] = static_cast<std::uint32_t>(q);
            }
        } else if (overflow != nullptr && (lds_overflow != 0u || in.reset_overflow)) {
            overflow[q] = lds_overflow != 0u ? 1u : 0u;
        }
    }
    __syncthreads();
    return lds.flagged != 0u;
}

}  // namespace

}  // namespace zcgvs_hip
