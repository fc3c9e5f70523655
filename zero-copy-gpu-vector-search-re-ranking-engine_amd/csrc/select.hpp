// Exact top-k selection on 64-bit keys (see common.hpp for the key layout).
//
// The k best keys of a set are found by a most-significant-digit radix select: histograms of
// successive digits (11, 11, 10 bits of the score, then 11, 11, 10 bits of the index part) narrow
// down the bucket that holds the k-th best key. Once a bucket's population equals the number of
// keys still needed, every key >= that bucket's lower edge is selected, which is exactly k keys
// because keys are unique. Each selected key then goes to its rank in descending order.
#pragma once

#include "common.hpp"

namespace zcgvs_hip {

constexpr int kSelectBins = 2048;
constexpr int kSelectPasses = 6;
constexpr int kSelectThreads = 256;
constexpr int kMergeThreads = 1024;  // block size of the fused search's per-query merge
constexpr int kMaxK = 1024;

__host__ __device__ constexpr int selectDigitWidth(int pass) {
    return (pass % 3 == 2) ? 10 : 11;
}

// Bits of the key decided before `pass`.
__host__ __device__ constexpr int selectBitsBefore(int pass) {
    return pass == 0 ? 0 : pass == 1 ? 11 : pass == 2 ? 22 : pass == 3 ? 32 : pass == 4 ? 43 : 54;
}

struct SelectState {
    std::uint64_t prefix;  // decided high bits, right-aligned
    std::uint32_t bits;    // number of decided bits
    std::uint32_t need;    // keys still to take from inside the prefix bucket
    std::uint32_t done;    // threshold is final
    std::uint32_t arrived; // blocks finished with the current pass (multi-block form)
    std::uint32_t count;   // keys collected
    std::uint32_t pad;
};

__device__ __forceinline__ std::uint64_t selectThreshold(const SelectState& s) {
    return s.bits >= 64 ? s.prefix : (s.prefix << (64 - s.bits));
}

// Inclusive sum over the 64 lanes of a wavefront (lanes 0..l) with data-parallel moves: a
// Hillis-Steele scan inside each 16-lane row (row shifts by 1, 2, 4, 8; lanes shifted in from
// outside the row read 0), then lane 15 of each row is added to the next row and lane 31 to the
// upper half. All lanes must be active.
__device__ __forceinline__ std::uint32_t waveInclusiveSum(std::uint32_t value) {
    int v = static_cast<int>(value);
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);  // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15 into rows 1, 3
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31 into rows 2, 3
    return static_cast<std::uint32_t>(v);
}

// Inclusive sum of `value` over the block's threads in thread order (threads 0..t), for a block
// of kThreads threads: a wavefront scan, then the wavefront totals through LDS (`wave_sums`,
// kThreads / kWave words). `total` receives the block's sum. Two barriers; every thread must
// call it.
template <int kThreads = kSelectThreads>
__device__ inline std::uint32_t blockInclusiveSum(std::uint32_t value, std::uint32_t* wave_sums,
                                                  std::uint32_t* total) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    value = waveInclusiveSum(value);
    if (lane == kWave - 1) {
        wave_sums[wave] = value;
    }
    __syncthreads();
    std::uint32_t before = 0u;
    std::uint32_t sum = 0u;
#pragma unroll
    for (int w = 0; w < kThreads / kWave; ++w) {
        const std::uint32_t v = wave_sums[w];
        before += w < wave ? v : 0u;
        sum += v;
    }
    __syncthreads();  // wave_sums is free again
    *total = sum;
    return value + before;
}

// Given a full histogram of the current digit, pick the bucket holding the need-th best key and
// update the state. Runs on one block of kThreads threads (at most 1024); `scratch` is LDS of
// kThreads / kWave u32. The histogram may be in LDS or global memory (read with plain loads; the
// caller makes it visible first).
template <int kThreads = kSelectThreads>
__device__ inline void selectPickBucket(const std::uint32_t* hist, int width, SelectState* state,
                                        std::uint32_t* scratch) {
    const int bins = 1 << width;
    const int per_thread = (bins + kThreads - 1) / kThreads;  // 8 or 4 at 256 threads, 2 or 1 at 1024
    const int t = threadIdx.x;
    // Thread t owns the t-th group of bins counted from the top (none once they run out).
    const int top = bins - per_thread * t;  // exclusive upper bin
    const int bottom = max(0, top - per_thread);
    std::uint32_t local = 0;
    for (int b = top - 1; b >= bottom; --b) {
        local += hist[b];
    }
    const std::uint32_t need = state->need;
    std::uint32_t total = 0u;
    const std::uint32_t through = blockInclusiveSum<kThreads>(local, scratch, &total);
    const std::uint32_t before = through - local;
    if (before < need && need <= through) {
        std::uint32_t above = before;
        for (int b = top - 1; b >= bottom; --b) {
            const std::uint32_t h = hist[b];
            if (above + h >= need) {
                const std::uint32_t remaining = need - above;
                state->prefix = (state->prefix << width) | static_cast<std::uint64_t>(b);
                state->bits += static_cast<std::uint32_t>(width);
                state->need = remaining;
                state->done = (h == remaining || state->bits >= 64) ? 1u : 0u;
                break;
            }
            above += h;
        }
    }
    __syncthreads();
}

// Visits the `count` keys of `keys` (in LDS, unique apart from repeated zero keys) with their
// rank in descending order, the number of keys above them: key i belongs at position
// #{j : keys[j] > keys[i]} of the sorted list. One pass of count comparisons per key (every lane
// reads the same key, an LDS broadcast) and no barrier replace a sorting network.
template <typename F>
__device__ inline void forEachRanked(const std::uint64_t* keys, std::uint32_t count, F&& f) {
    for (std::uint32_t i = threadIdx.x; i < count; i += blockDim.x) {
        const std::uint64_t key = keys[i];
        std::uint32_t rank = 0u;
#pragma unroll 8
        for (std::uint32_t j = 0; j < count; ++j) {
            rank += keys[j] > key ? 1u : 0u;
        }
        f(rank, key);
    }
}

// ---- host-side internal API used by the fused search -----------------------------------------

// Inputs of one per-query merge. For query q the candidate set is the union of
//   prev[q][0..k_prev)                       the selection kept from earlier phases,
//   dense[q * dense_stride + 0..n_dense)     keys written at fixed slots (key 0 = empty slot),
//   seg[((s * batch + q) << seg_log2) + j]   for every segment s < n_seg and
//                                            j < min(seg_count[s * batch + q], 1 << seg_log2),
// where each segment is the private append buffer of one workgroup of a scan launch.
struct MergeInputs {
    const std::uint64_t* prev = nullptr;
    int k_prev = 0;
    const std::uint64_t* dense = nullptr;
    long long n_dense = 0;
    long long dense_stride = 0;
    const std::uint64_t* seg = nullptr;
    const std::uint32_t* seg_count = nullptr;
    int n_seg = 0;
    int seg_log2 = 0;
    // true for the first merge of a search: it writes every query's overflow flag (0 or 1)
    // instead of only raising flags, so no separate clearing pass is needed
    bool reset_overflow = false;
    // When set (first merge of a phased search), block 0 clears *zero_count: the exact
    // fallback's list of flagged queries starts empty.
    std::uint32_t* zero_count = nullptr;
    // The search's last merge flags a query for the exact fallback when a segment overflowed in
    // this or an earlier phase (the overflow flag an earlier merge raised), or, with
    // require_full, when fewer than k keys reached it (a speculative threshold was above the
    // k-th best key). A flagged query gets overflow[q] = 1, is appended to flag_list (length in
    // *flag_count) and gets the fallback's threshold in rerun_tau[q]: its k-th best key minus
    // one when it has k keys (every key >= that k-th best key passes), else fallback_tau[q] (a
    // guaranteed lower bound; 0 without one). Other queries get overflow[q] = 0.
    bool final_merge = false;
    bool require_full = false;
    const std::uint64_t* fallback_tau = nullptr;
    std::uint32_t* flag_list = nullptr;
    std::uint32_t* flag_count = nullptr;
    std::uint64_t* rerun_tau = nullptr;
};

// Selects the best k keys of each query's candidate set; writes them to out_keys[q][0..k)
// (sorted descending when out_index is set, in no particular order otherwise; missing keys are
// 0 at the end), sets threshold[q] to the k-th best key (0 if fewer than k keys exist) and
// sets overflow[q] when a segment count exceeded its capacity (and clears it otherwise when
// in.reset_overflow is set). When out_index/out_score are
// non-null the selection is also written as (index, score) pairs [batch, k].
int launchSelectMerge(const MergeInputs& in, int k, int batch, std::uint64_t* out_keys,
                      std::uint64_t* threshold, std::uint32_t* overflow, int* out_index,
                      float* out_score, hipStream_t stream);

// The same selection (segments only, no threshold) for candidate segments that each hold at most
// k keys sorted descending, as the single-pass scan writes them: the k-th best segment head bounds
// the result from below, so only the segments whose head reaches it (at most k) are read past
// their first key. For k <= kSortedSelectMaxK and n_seg <= kSortedMergeMaxSegments: up to
// kSortedMergeMaxK the candidates are ranked by comparison, above it the best k of them are first
// selected by radix passes in LDS (k * k candidates at most).
constexpr int kSortedMergeMaxK = 32;
constexpr int kSortedSelectMaxK = 110;  // 110 * 110 candidates fit the merge's 12288 LDS keys
constexpr int kSortedMergeMaxSegments = 1024;
int launchSortedSegmentMerge(const MergeInputs& in, int k, int batch, std::uint64_t* out_keys,
                             std::uint32_t* overflow, int* out_index, float* out_score, hipStream_t stream);

// Thresholds of a speculative scan from a sketch phase (one block per query). Slot s holds the
// best exact score of its rows, sketch[s * batch + q] (-inf: the slot saw no row); the slots'
// rows are disjoint, so their scores belong to distinct corpus rows. tau[q] admits every score
// >= the j-th best slot score and tau_safe[q] every score >= the k-th best one (as the keys
// ordered32(score) << 32; 0 = no threshold when fewer slots hold a score). tau_safe is a lower
// bound of the k-th best key of the corpus; tau is only likely to be one. Block 0 also clears
// *flag_count.
constexpr int kMaxSketchSlots = 2048;
int launchSketchThreshold(const float* sketch, int slots, int batch, int j, int k, std::uint64_t* tau,
                          std::uint64_t* tau_safe, std::uint32_t* flag_count, hipStream_t stream);

}  // namespace zcgvs_hip
