// Hybrid lexical stage: BM25 over CSR postings (src/cuda/lexical.cu:17-42, 78-92), the
// per-query positive maximum (lexical.cu:44-65, 94-105) and the convex fusion with the dense
// score (lexical.cu:67-74, 107-123).
//
// Determinism. The reference launches one block per query term and scatter-adds with float
// atomics, so a document hit by several terms sums them in a run-dependent order. Here the term
// slots of a query are processed one launch at a time, in slot order; inside a launch the
// postings of one term touch distinct documents (the index builder emits one posting per
// (term, document)), so every document's sum is ((w_0 + w_1) + w_2) ... in slot order, the order
// of the CPU loop in tests/cpp/test_lexical.cu:71-80, on every run.
//
// The fused search's default needs no atomics in global memory and no separate clearing or
// maximum pass. With every term's postings ascending by document, bm25BoundsKernel finds where
// each query term's postings cross every 4096-document boundary (one binary search per thread,
// all at once), and bm25SweepKernel, one workgroup per (query, slice), loads its slice of every
// term's postings, adds them into an LDS accumulator slot by slot in slot order (the same
// per-document order), then writes the slice, zeros included, and folds its maximum into the
// query's. An index may also carry a slice table (built once, zcgvs_build_lexical_slice_table):
// for every term, the number of its postings below each 4096-document boundary, so a search
// gathers its terms' slice bounds from it (two loads) instead of binary-searching the postings
// (about twenty dependent loads per bound).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.hpp"
#include "rescore.hpp"

namespace zcgvs_hip {

namespace {

constexpr int kPostingThreads = 256;
constexpr int kReduceThreads = 256;
constexpr int kSweepThreads = 512;
// documents per sweep workgroup (measured on the 1M-document hybrid search, BM25 stage: 1024
// documents and 256 threads 114 us, 2048 and 256 threads 105 us, 4096 and 512 threads 100 us;
// 4096 and 256, 8192 and 1024, or one slot per load group are slower)
constexpr int kSweepDocs = 4096;
constexpr int kSweepPerThread = kSweepDocs / kSweepThreads;  // postings per thread per slot
// slots whose postings are loaded together: two keep the sweep at about 40 registers, so more
// (query, slice) workgroups are resident to hide each other's load latency (measured: 8 slots
// 0.32 ms per hybrid search, 4 slots 0.31 ms, 2 slots 0.30 ms, 1 slot 0.31 ms)
constexpr int kSweepSlotGroup = 2;
// Workgroups go to the XCDs (each with its own L2) round-robin in launch order; the sweep keeps
// every query of a slice on one XCD (see bm25SweepKernel).
constexpr int kXcds = 8;

// Postings of term slot `slot` for each query (blockIdx.y) of the batch.
__global__ __launch_bounds__(kPostingThreads) void bm25SlotKernel(
    const std::int64_t* __restrict__ offsets, const int* __restrict__ docs,
    const float* __restrict__ weights, const int* __restrict__ query_terms, int term_stride,
    int slot, int doc_count, int vocab_size, float* __restrict__ scores) {
    const int q = blockIdx.y;
    const int term = query_terms[static_cast<std::size_t>(q) * term_stride + slot];
    if (term < 0 || term >= vocab_size) {
        return;
    }
    const std::int64_t begin = offsets[term];
    const std::int64_t end = offsets[term + 1];
    float* row = scores + static_cast<std::size_t>(q) * doc_count;
    for (std::int64_t p = begin + static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
         p < end; p += static_cast<std::int64_t>(gridDim.x) * blockDim.x) {
        const int doc = docs[p];
        if (doc >= 0 && doc < doc_count) {
            atomicAdd(&row[doc], weights[p]);
        }
    }
}

// Raises *target (a non-negative float, ordered as its bits) to at least `value`. Thousands of
// workgroups fold into one address per query, and atomics on one address serialize, so the
// current value is read first and the atomic is issued only when it would raise it (a stale
// read only costs an unneeded atomic).
__device__ __forceinline__ void raiseMax(float* target, float value) {
    unsigned int* bits = reinterpret_cast<unsigned int*>(target);
    const unsigned int mine = __float_as_uint(value);
    if (__atomic_load_n(bits, __ATOMIC_RELAXED) < mine) {
        atomicMax(bits, mine);
    }
}

// First position in docs[lo, hi) whose document is >= target (hi if none).
__device__ __forceinline__ std::int64_t lowerBound(const int* __restrict__ docs, std::int64_t lo,
                                                   std::int64_t hi, int target) {
    while (lo < hi) {
        const std::int64_t mid = lo + ((hi - lo) >> 1);
        if (docs[mid] < target) {
            lo = mid + 1;
        } else {
            hi = mid;
        }
    }
    return lo;
}

// table[t * table_stride + c] = the number of term t's postings whose document is below
// c * kSweepDocs (c = table_stride - 1: below the index's doc_count). One thread per entry.
__global__ void sliceTableKernel(const std::int64_t* __restrict__ offsets, const int* __restrict__ docs,
                                 int vocab_size, std::int64_t doc_count, int table_stride,
                                 std::uint32_t* __restrict__ table) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<long long>(vocab_size) * table_stride) {
        return;
    }
    const int c = static_cast<int>(i % table_stride);
    const int term = static_cast<int>(i / table_stride);
    const std::int64_t lo = offsets[term];
    const long long target = c == table_stride - 1 ? doc_count : static_cast<long long>(c) * kSweepDocs;
    const int bound = static_cast<int>(min(target, static_cast<long long>(INT32_MAX)));
    table[i] = static_cast<std::uint32_t>(lowerBound(docs, lo, offsets[term + 1], bound) - lo);
}

// bounds[(q * term_stride + slot) * (slices + 1) + c] = first posting of the term in slot `slot`
// of query q whose document is >= c * kSweepDocs (c = slices: >= doc_count); an unknown term
// gets 0 everywhere (an empty range). One thread per entry, so all searches run at once. With
// a slice table the entry is gathered from it instead (for c = slices its count may include
// postings of documents from doc_count up to the index's own count, inside the last slice's
// document range; the sweep skips them). Also zeroes lexical_max[0, batch) (there are at least
// batch entries: slices + 1 >= 2, term_stride >= 1).
__global__ void bm25BoundsKernel(const std::int64_t* __restrict__ offsets, const int* __restrict__ docs,
                                 const int* __restrict__ query_terms, int term_stride, int batch,
                                 int doc_count, int vocab_size, int slices,
                                 const std::uint32_t* __restrict__ table, int table_stride,
                                 std::int64_t* __restrict__ bounds, float* __restrict__ lexical_max) {
    const long long total = static_cast<long long>(batch) * term_stride * (slices + 1);
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < batch) {
        lexical_max[i] = 0.0f;  // the sweep that follows raises it
    }
    if (i >= total) {
        return;
    }
    const int c = static_cast<int>(i % (slices + 1));
    const long long qs = i / (slices + 1);  // q * term_stride + slot
    const int term = query_terms[qs];
    std::int64_t position = 0;
    if (term >= 0 && term < vocab_size) {
        if (table != nullptr) {
            position = offsets[term] + table[static_cast<std::size_t>(term) * table_stride + c];
        } else {
            position = lowerBound(docs, offsets[term], offsets[term + 1],
                                  c == slices ? doc_count : c * kSweepDocs);
        }
    }
    bounds[i] = position;
}

// BM25 scores of documents [blockIdx.x * kSweepDocs, + kSweepDocs) for query blockIdx.y from the
// postings between the slice bounds; writes every score of the slice and raises lexical_max[q]
// (zeroed beforehand) to the slice's max(0, max score). A slot's postings inside one slice are
// distinct documents, so there are at most kSweepDocs of them: thread t loads the
// kSweepPerThread = 8 postings from begin + 8t with two 16-byte loads of documents and two of
// weights (a range's last thread starts at end - 8, so no load leaves the range; ranges under 8
// postings load them one by one),
// for kSweepSlotGroup slots at a time, before any is added, and the additions of one slot touch
// distinct accumulator entries.
//
// Queries share their frequent terms, whose postings cover most documents, so the launch's
// queries of one slice run back to back on one XCD: workgroup w runs on XCD w % kXcds as that
// XCD's (w / kXcds)-th, which takes query q_offset + (w / kXcds) % q_count of slice
// kXcds * ((w / kXcds) / q_count) + w % kXcds; the later queries then find the slice's shared
// postings in that XCD's L2. The grid has kXcds * ceil(slices / kXcds) * q_count workgroups.
__global__ __launch_bounds__(kSweepThreads) void bm25SweepKernel(
    const int* __restrict__ docs, const float* __restrict__ weights, const std::int64_t* __restrict__ bounds,
    int term_stride, int doc_count, int slices, int q_offset, int q_count, float* __restrict__ scores,
    float* __restrict__ lexical_max) {
    __shared__ __attribute__((aligned(16))) float acc[kSweepDocs];
    __shared__ float partial[kSweepThreads / kWave];
    const int xcd_rank = static_cast<int>(blockIdx.x / kXcds);
    const int q = q_offset + xcd_rank % q_count;
    const int c = kXcds * (xcd_rank / q_count) + static_cast<int>(blockIdx.x % kXcds);
    if (c >= slices) {
        return;
    }
    const int t = threadIdx.x;
    const int d0 = c * kSweepDocs;
    const int d1 = min(d0 + kSweepDocs, doc_count);
    for (int i = t; i < kSweepDocs; i += kSweepThreads) {
        acc[i] = 0.0f;
    }
    __syncthreads();
    const std::int64_t* qb = bounds + static_cast<std::size_t>(q) * term_stride * (slices + 1);
    for (int g0 = 0; g0 < term_stride; g0 += kSweepSlotGroup) {
        int doc[kSweepSlotGroup][kSweepPerThread];
        float weight[kSweepSlotGroup][kSweepPerThread];
        std::int64_t begin[kSweepSlotGroup];
        std::int64_t end[kSweepSlotGroup];
        int first[kSweepSlotGroup];  // this thread's postings are entries [first, last) of its load
        int last[kSweepSlotGroup];
#pragma unroll
        for (int g = 0; g < kSweepSlotGroup; ++g) {  // all bounds first: one wait for all of them
            const int slot = g0 + g;
            begin[g] = 0;
            end[g] = 0;
            if (slot < term_stride) {
                begin[g] = qb[static_cast<std::size_t>(slot) * (slices + 1) + c];
                end[g] = qb[static_cast<std::size_t>(slot) * (slices + 1) + c + 1];
            }
        }
        // Every load of the group is issued before any loaded value is used.
#pragma unroll
        for (int g = 0; g < kSweepSlotGroup; ++g) {
            const std::int64_t count = end[g] - begin[g];  // uniform over the workgroup
            const std::int64_t p = begin[g] + static_cast<std::int64_t>(kSweepPerThread) * t;
            first[g] = 0;
            last[g] = 0;
            if (count >= kSweepPerThread) {
                const std::int64_t from = p < end[g] - kSweepPerThread ? p : end[g] - kSweepPerThread;
                __builtin_memcpy(&doc[g][0], docs + from, sizeof(doc[g]));
                __builtin_memcpy(&weight[g][0], weights + from, sizeof(weight[g]));
                first[g] = static_cast<int>(p - from);
                last[g] = static_cast<int>(min(end[g], p + kSweepPerThread) - from);
            } else if (count > 0) {
#pragma unroll
                for (int j = 0; j < kSweepPerThread; ++j) {
                    const std::int64_t at = begin[g] + j < end[g] ? begin[g] + j : end[g] - 1;
                    doc[g][j] = docs[at];
                    weight[g][j] = weights[at];
                }
                last[g] = t == 0 ? static_cast<int>(count) : 0;
            }
        }
#pragma unroll
        for (int g = 0; g < kSweepSlotGroup; ++g) {
            if (g0 + g < term_stride) {
                if (end[g] > begin[g]) {
#pragma unroll
                    for (int j = 0; j < kSweepPerThread; ++j) {
                        // distinct documents within a slot: plain adds do not race (and an
                        // LDS float atomic is several times slower here)
                        if (j >= first[g] && j < last[g] && doc[g][j] >= d0 && doc[g][j] < d1) {
                            acc[doc[g][j] - d0] += weight[g][j];
                        }
                    }
                    // More than kSweepDocs postings in one slice can only come from repeated
                    // documents, which the sorted-postings contract excludes: their additions
                    // race with the plain adds above, so such an index gives undefined sums
                    // (the caller states the contract with ZCGVS_SEARCH_SORTED_POSTINGS).
                    for (std::int64_t p = begin[g] + kSweepDocs + t; p < end[g]; p += kSweepThreads) {
                        const int extra = docs[p];
                        if (extra >= d0 && extra < d1) {
                            atomicAdd(&acc[extra - d0], weights[p]);
                        }
                    }
                }
                __syncthreads();  // slot g's additions land before slot g + 1's
            }
        }
    }
    float best = 0.0f;
    float* row = scores + static_cast<std::size_t>(q) * doc_count + d0;
    if (d1 - d0 == kSweepDocs && (reinterpret_cast<std::uintptr_t>(row) & 15u) == 0) {
#pragma unroll
        for (int i = t; i < kSweepDocs / 4; i += kSweepThreads) {
            const float4 value = reinterpret_cast<const float4*>(acc)[i];
            reinterpret_cast<float4*>(row)[i] = value;
            best = fmaxf(best, fmaxf(fmaxf(value.x, value.y), fmaxf(value.z, value.w)));
        }
    } else {
        for (int i = t; i < d1 - d0; i += kSweepThreads) {
            const float value = acc[i];
            row[i] = value;
            best = fmaxf(best, value);
        }
    }
    best = fmaxf(best, 0.0f);
#pragma unroll
    for (int offset = kWave / 2; offset > 0; offset >>= 1) {
        best = fmaxf(best, waveXor(best, offset));
    }
    if ((t & (kWave - 1)) == 0) {
        partial[t / kWave] = best;
    }
    __syncthreads();
    if (t == 0) {
        float block_best = 0.0f;
        for (int w = 0; w < kSweepThreads / kWave; ++w) {
            block_best = fmaxf(block_best, partial[w]);
        }
        raiseMax(lexical_max + q, block_best);
    }
}

// max(0, max_i values[q][i]) folded into out_max[q] with an unsigned max on the float bits,
// which orders non-negative floats correctly (lexical.cu:61-63).
__global__ __launch_bounds__(kReduceThreads) void maxPositiveKernel(
    const float* __restrict__ values, int count, float* __restrict__ out_max) {
    __shared__ float partial[kReduceThreads / kWave];
    const int q = blockIdx.y;
    const float* row = values + static_cast<std::size_t>(q) * count;
    float best = 0.0f;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += gridDim.x * blockDim.x) {
        best = fmaxf(best, row[i]);
    }
#pragma unroll
    for (int offset = kWave / 2; offset > 0; offset >>= 1) {
        best = fmaxf(best, waveXor(best, offset));
    }
    if ((threadIdx.x & (kWave - 1)) == 0) {
        partial[threadIdx.x / kWave] = best;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float block_best = 0.0f;
        for (int w = 0; w < kReduceThreads / kWave; ++w) {
            block_best = fmaxf(block_best, partial[w]);
        }
        raiseMax(out_max + q, block_best);
    }
}

// dense = w * dense + (1 - w) * lexical * inverse, with inverse = 1/max or 0, evaluated as
// separate IEEE multiplies and adds in the reference's operand order.
__global__ __launch_bounds__(kReduceThreads) void fuseScoresKernel(
    float* __restrict__ dense, const float* __restrict__ lexical,
    const float* __restrict__ lexical_max, float weight, int count) {
#pragma clang fp contract(off)
    const float peak = *lexical_max;
    const float inverse = (peak > 0.0f) ? (1.0f / peak) : 0.0f;
    const float lexical_weight = 1.0f - weight;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += gridDim.x * blockDim.x) {
        const float a = weight * dense[i];
        const float b = lexical_weight * lexical[i];
        const float c = b * inverse;
        dense[i] = a + c;
    }
}

__global__ void zeroKernel(float* __restrict__ dst, std::size_t count) {
    const std::size_t stride = static_cast<std::size_t>(gridDim.x) * blockDim.x;
    for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
         i < count; i += stride) {
        dst[i] = 0.0f;
    }
}

unsigned reduceBlocks(long long count) {
    long long blocks = (count + kReduceThreads - 1) / kReduceThreads;
    return static_cast<unsigned>(std::max(1LL, std::min(blocks, 256LL)));
}

unsigned postingBlocks() { return static_cast<unsigned>(std::max(1, deviceComputeUnits())); }

}  // namespace

std::size_t lexicalBoundsBytes(int batch, int term_stride, int doc_count) {
    const long long slices = (static_cast<long long>(doc_count) + kSweepDocs - 1) / kSweepDocs;
    return static_cast<std::size_t>(batch) * static_cast<std::size_t>(term_stride) *
           static_cast<std::size_t>(slices + 1) * sizeof(std::int64_t);
}

int lexicalSliceTableStride(std::int64_t doc_count) {
    return static_cast<int>((doc_count + kSweepDocs - 1) / kSweepDocs) + 1;
}

int launchLexicalScores(const std::int64_t* offsets, const int* docs, const float* weights,
                        int vocab_size, const int* query_terms, int term_stride, int batch,
                        int doc_count, float* lexical, float* lexical_max, std::int64_t* bounds,
                        const std::uint32_t* slice_table, std::int64_t index_doc_count,
                        hipStream_t stream) {
    if (bounds != nullptr) {
        const int slices = (doc_count + kSweepDocs - 1) / kSweepDocs;
        const long long entries = static_cast<long long>(batch) * term_stride * (slices + 1);
        const int table_stride = slice_table != nullptr ? lexicalSliceTableStride(index_doc_count) : 0;
        bm25BoundsKernel<<<static_cast<unsigned>((entries + 255) / 256), 256, 0, stream>>>(
            offsets, docs, query_terms, term_stride, batch, doc_count, vocab_size, slices, slice_table,
            table_stride, bounds, lexical_max);
        ZCGVS_LAUNCH_CHECK("bm25 bounds");
        // queries per launch: the grid's threads stay below 2^31
        const long long per_query = static_cast<long long>((slices + kXcds - 1) / kXcds) * kXcds;
        const int chunk = static_cast<int>(std::max<long long>(
            1, std::min<long long>(batch, (1LL << 31) / (per_query * kSweepThreads))));
        for (int q0 = 0; q0 < batch; q0 += chunk) {
            const int count = std::min(chunk, batch - q0);
            bm25SweepKernel<<<static_cast<unsigned>(per_query * count), kSweepThreads, 0, stream>>>(
                docs, weights, bounds, term_stride, doc_count, slices, q0, count, lexical, lexical_max);
        }
        ZCGVS_LAUNCH_CHECK("bm25 sweep");
        return ZCGVS_OK;
    }
    zeroKernel<<<1, 256, 0, stream>>>(lexical_max, static_cast<std::size_t>(batch));
    ZCGVS_LAUNCH_CHECK("lexical zero");
    const std::size_t elements = static_cast<std::size_t>(batch) * doc_count;
    zeroKernel<<<std::min<std::size_t>(8192, (elements + 255) / 256), 256, 0, stream>>>(lexical, elements);
    ZCGVS_LAUNCH_CHECK("lexical zero");
    const dim3 grid(postingBlocks(), static_cast<unsigned>(batch));
    for (int slot = 0; slot < term_stride; ++slot) {
        bm25SlotKernel<<<grid, kPostingThreads, 0, stream>>>(offsets, docs, weights, query_terms,
                                                             term_stride, slot, doc_count,
                                                             vocab_size, lexical);
    }
    ZCGVS_LAUNCH_CHECK("bm25");
    maxPositiveKernel<<<dim3(reduceBlocks(doc_count), static_cast<unsigned>(batch)),
                        kReduceThreads, 0, stream>>>(lexical, doc_count, lexical_max);
    ZCGVS_LAUNCH_CHECK("lexical max");
    return ZCGVS_OK;
}

}  // namespace zcgvs_hip

using namespace zcgvs_hip;

extern "C" {

int zcgvs_launch_bm25(const std::int64_t* d_offsets, const int* d_docs, const float* d_weights,
                      const int* d_query_terms, int term_count, int doc_count, float* d_scores,
                      zcgvs_stream_t stream) {
    if (term_count <= 0 || doc_count <= 0) {
        return clearError();
    }
    return zcgvs_launch_bm25_batched(d_offsets, d_docs, d_weights, d_query_terms, term_count, 1,
                                     doc_count, d_scores, stream);
}

int zcgvs_launch_bm25_batched(const std::int64_t* d_offsets, const int* d_docs,
                              const float* d_weights, const int* d_query_terms, int term_stride,
                              int batch, int doc_count, float* d_scores, zcgvs_stream_t stream) {
    if (term_stride <= 0 || doc_count <= 0 || batch <= 0) {
        return clearError();
    }
    if (d_offsets == nullptr || d_query_terms == nullptr || d_scores == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs bm25: null device pointer");
    }
    const dim3 grid(postingBlocks(), static_cast<unsigned>(batch));
    for (int slot = 0; slot < term_stride; ++slot) {
        bm25SlotKernel<<<grid, kPostingThreads, 0, toStream(stream)>>>(
            d_offsets, d_docs, d_weights, d_query_terms, term_stride, slot, doc_count, INT32_MAX,
            d_scores);
    }
    ZCGVS_LAUNCH_CHECK("bm25");
    return clearError();
}

size_t zcgvs_lexical_slice_table_bytes(int vocab_size, int64_t doc_count) {
    if (vocab_size <= 0 || doc_count <= 0 || doc_count > INT32_MAX) {
        return 0;
    }
    return static_cast<std::size_t>(vocab_size) * static_cast<std::size_t>(lexicalSliceTableStride(doc_count)) *
           sizeof(std::uint32_t);
}

int zcgvs_build_lexical_slice_table(const int64_t* d_offsets, const int* d_docs, int vocab_size,
                                    int64_t doc_count, uint32_t* d_table, zcgvs_stream_t stream) {
    if (vocab_size <= 0 || doc_count <= 0 || doc_count > INT32_MAX) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs slice table: empty index or too many documents");
    }
    if (d_offsets == nullptr || d_docs == nullptr || d_table == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs slice table: null device pointer");
    }
    const int stride = lexicalSliceTableStride(doc_count);
    const long long entries = static_cast<long long>(vocab_size) * stride;
    if (entries > (1LL << 31) - 256) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs slice table: too many entries for one launch");
    }
    sliceTableKernel<<<static_cast<unsigned>((entries + 255) / 256), 256, 0, toStream(stream)>>>(
        d_offsets, d_docs, vocab_size, doc_count, stride, d_table);
    ZCGVS_LAUNCH_CHECK("slice table");
    return clearError();
}

int zcgvs_launch_max_positive(const float* d_values, int count, float* d_max,
                              zcgvs_stream_t stream) {
    if (count <= 0) {
        return clearError();
    }
    if (d_values == nullptr || d_max == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs max: null device pointer");
    }
    maxPositiveKernel<<<dim3(reduceBlocks(count), 1), kReduceThreads, 0, toStream(stream)>>>(
        d_values, count, d_max);
    ZCGVS_LAUNCH_CHECK("max positive");
    return clearError();
}

int zcgvs_launch_fuse_scores(float* d_dense, const float* d_lexical, const float* d_lexical_max,
                             float weight, int count, zcgvs_stream_t stream) {
    if (count <= 0) {
        return clearError();
    }
    if (d_dense == nullptr || d_lexical == nullptr || d_lexical_max == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs fuse: null device pointer");
    }
    fuseScoresKernel<<<reduceBlocks(count), kReduceThreads, 0, toStream(stream)>>>(
        d_dense, d_lexical, d_lexical_max, weight, count);
    ZCGVS_LAUNCH_CHECK("fuse");
    return clearError();
}

}  // extern "C"
