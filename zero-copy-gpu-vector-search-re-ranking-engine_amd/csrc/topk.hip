// Top-k selection: zcgvs_launch_topk (src/cuda/topk.cu:132-189 launchTopK) over a materialized
// [batch, doc_count] score matrix, and the per-query candidate merge used by the fused search.
//
// The reference sorts 1024-score tiles with a bitonic network and merges tile winners
// recursively; ties fall wherever the network puts them. Here the selection is an exact radix
// select on unique 64-bit keys (select.hpp), so the result is the stable (score desc, index asc)
// order of tests/cpp/cpu_reference.hpp:26-34 on every run. Each pass reads the scores once; the
// block that finishes a pass last picks the bucket (no host round trip, capture safe).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.hpp"
#include "merge.hpp"
#include "select.hpp"

namespace zcgvs_hip {

namespace {

constexpr int kTileSize = 1024;      // reference tile (topk.cu:17), kept for the sizing helpers
constexpr int kMergeTile = 4096;     // reference merge tile (topk.cu:18)
constexpr int kStateWords = 16;      // SelectState, padded
constexpr int kMinScratchElements = kStateWords + kSelectBins + 16;

struct TopKScratch {
    __host__ __device__ SelectState* state(int q) const {
        return reinterpret_cast<SelectState*>(base + static_cast<std::size_t>(q) * stride);
    }
    __host__ __device__ std::uint32_t* hist(int q) const {
        return base + static_cast<std::size_t>(q) * stride + kStateWords;
    }
    std::uint32_t* base;
    std::size_t stride;  // u32 words per query
};

struct KeyScratch {
    __host__ __device__ std::uint64_t* keys(int q) const {
        return reinterpret_cast<std::uint64_t*>(base + static_cast<std::size_t>(q) * stride);
    }
    std::uint32_t* base;
    std::size_t stride;  // u32 words per query (even)
};

__global__ void topkInitKernel(TopKScratch scratch, int k) {
    const int q = blockIdx.x;
    std::uint32_t* hist = scratch.hist(q);
    for (int i = threadIdx.x; i < kSelectBins; i += blockDim.x) {
        hist[i] = 0u;
    }
    if (threadIdx.x == 0) {
        SelectState* s = scratch.state(q);
        s->prefix = 0ull;
        s->bits = 0u;
        s->need = static_cast<std::uint32_t>(k);
        s->done = 0u;
        s->arrived = 0u;
        s->count = 0u;
    }
}

__global__ __launch_bounds__(kSelectThreads) void topkHistKernel(const float* __restrict__ scores,
                                                                 int doc_count, int pass,
                                                                 TopKScratch scratch) {
    __shared__ std::uint32_t lds_hist[kSelectBins];
    __shared__ std::uint32_t lds_scan[kSelectThreads];
    __shared__ SelectState lds_state;
    __shared__ int is_last;

    const int q = blockIdx.y;
    SelectState* state = scratch.state(q);
    if (threadIdx.x == 0) {
        lds_state = *state;
    }
    for (int i = threadIdx.x; i < kSelectBins; i += blockDim.x) {
        lds_hist[i] = 0u;
    }
    __syncthreads();
    if (lds_state.done) {
        return;
    }
    const int width = selectDigitWidth(pass);
    const std::uint32_t bits = lds_state.bits;
    const std::uint64_t prefix = lds_state.prefix;
    const int shift = 64 - static_cast<int>(bits) - width;
    const std::uint64_t digit_mask = (1ull << width) - 1ull;
    const float* row = scores + static_cast<std::size_t>(q) * doc_count;
    for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
         i < doc_count; i += static_cast<long long>(gridDim.x) * blockDim.x) {
        const std::uint64_t key = makeKey(row[i], static_cast<std::uint32_t>(i));
        if (bits == 0u || (key >> (64 - bits)) == prefix) {
            atomicAdd(&lds_hist[(key >> shift) & digit_mask], 1u);
        }
    }
    __syncthreads();
    std::uint32_t* hist = scratch.hist(q);
    for (int b = threadIdx.x; b < (1 << width); b += blockDim.x) {
        if (lds_hist[b] != 0u) {
            atomicAdd(&hist[b], lds_hist[b]);
        }
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const std::uint32_t ticket = atomicAdd(&state->arrived, 1u);
        is_last = (ticket == gridDim.x - 1) ? 1 : 0;
    }
    __syncthreads();
    if (!is_last) {
        return;
    }
    __threadfence();
    for (int b = threadIdx.x; b < (1 << width); b += blockDim.x) {
        lds_hist[b] = __hip_atomic_load(&hist[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        hist[b] = 0u;
    }
    __syncthreads();
    selectPickBucket(lds_hist, width, &lds_state, lds_scan);
    if (threadIdx.x == 0) {
        lds_state.arrived = 0u;
        *state = lds_state;
    }
    __threadfence();
}

__global__ __launch_bounds__(kSelectThreads) void topkCollectKernel(
    const float* __restrict__ scores, int doc_count, int k, TopKScratch scratch, KeyScratch out) {
    const int q = blockIdx.y;
    SelectState* state = scratch.state(q);
    const std::uint64_t threshold = selectThreshold(*state);
    std::uint64_t* keys = out.keys(q);
    const float* row = scores + static_cast<std::size_t>(q) * doc_count;
    for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
         i < doc_count; i += static_cast<long long>(gridDim.x) * blockDim.x) {
        const std::uint64_t key = makeKey(row[i], static_cast<std::uint32_t>(i));
        if (key >= threshold) {
            const std::uint32_t slot = atomicAdd(&state->count, 1u);
            if (slot < static_cast<std::uint32_t>(k)) {  // exactly k keys pass; guard anyway
                keys[slot] = key;
            }
        }
    }
}

__global__ __launch_bounds__(kSelectThreads) void topkSortKernel(TopKScratch scratch,
                                                                 KeyScratch in, int k,
                                                                 int* __restrict__ out_index,
                                                                 float* __restrict__ out_score) {
    __shared__ std::uint64_t lds_keys[kMaxK];
    const int q = blockIdx.x;
    const std::uint32_t count = min(min(scratch.state(q)->count, static_cast<std::uint32_t>(kMaxK)),
                                    static_cast<std::uint32_t>(k));
    const std::uint64_t* keys = in.keys(q);
    for (std::uint32_t i = threadIdx.x; i < count; i += blockDim.x) {
        lds_keys[i] = keys[i];
    }
    __syncthreads();
    forEachRanked(lds_keys, count, [&](std::uint32_t rank, std::uint64_t key) {
        const std::size_t o = static_cast<std::size_t>(q) * k + rank;
        writeHit(key, &out_index[o], &out_score[o]);
    });
    for (int i = static_cast<int>(count) + threadIdx.x; i < k; i += blockDim.x) {
        const std::size_t o = static_cast<std::size_t>(q) * k + i;
        writeHit(0ull, &out_index[o], &out_score[o]);
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
    const std::size_t elements = static_cast<std::size_t>(topkScratchElements(doc_count, k));
    TopKScratch scratch{reinterpret_cast<std::uint32_t*>(d_scratch_values_a), elements & ~std::size_t(1)};
    KeyScratch keys{reinterpret_cast<std::uint32_t*>(d_scratch_indices_a), elements & ~std::size_t(1)};
    const hipStream_t s = toStream(stream);

    const long long per_query_blocks = (static_cast<long long>(doc_count) + 8191) / 8192;
    const long long budget = std::max(1LL, 4LL * deviceComputeUnits() / batch);
    const unsigned tiles = static_cast<unsigned>(std::max(1LL, std::min(per_query_blocks, budget)));
    const dim3 grid(tiles, static_cast<unsigned>(batch));

    topkInitKernel<<<batch, kSelectThreads, 0, s>>>(scratch, k);
    ZCGVS_LAUNCH_CHECK("top-k init");
    for (int pass = 0; pass < kSelectPasses; ++pass) {
        topkHistKernel<<<grid, kSelectThreads, 0, s>>>(d_scores, doc_count, pass, scratch);
        ZCGVS_LAUNCH_CHECK("top-k histogram");
    }
    topkCollectKernel<<<grid, kSelectThreads, 0, s>>>(d_scores, doc_count, k, scratch, keys);
    ZCGVS_LAUNCH_CHECK("top-k collect");
    topkSortKernel<<<batch, kSelectThreads, 0, s>>>(scratch, keys, k, d_out_indices, d_out_values);
    ZCGVS_LAUNCH_CHECK("top-k sort");
    return clearError();
}

}  // extern "C"
