// Exact device fallback of the fused search: the top-`width` of one query over the whole corpus,
// for the queries the search's last merge flagged (a candidate segment overflowed, or a
// speculative threshold let fewer than width keys through), or for every query with
// ZCGVS_SEARCH_FORCE_EXACT_PASS.
//
// Sketch-planned searches: the scan kernel reran the flagged queries over the whole corpus, by
// every workgroup of the GPU, with a threshold that is a lower bound of their width-th best key
// and the batch's whole segment buffer shared among them; recoverKernel (one 1024-thread
// workgroup per list entry, the entries past the list returning at once) takes each query's
// selection from its rerun segments (radix passes over at most a few thousand keys). Other
// searches: mergeRecoverKernel runs the last merge and, in the same block, the last resort for a
// query that merge flags, so no separate launch runs when nothing is flagged.
//
// The last resort (a rerun segment overflowed too, the force flag, or a threshold-phase search):
// one workgroup sweeps the corpus once in index order, keeps every key above a running
// threshold in an LDS list and cuts the list to its width best keys whenever it could fill, so
// the list always holds the exact top-width of the rows swept so far. Keys are unique (score,
// then index), so this is the lowest-index tie rule of tests/cpp/cpu_reference.hpp:26-34. Its
// cost is one corpus read at the rate of one compute unit.
//
// Scores are computed as the VALU scan computes them (same lanes per row, chunk order and lane
// group sums, scan_core.hpp), so for every kind they equal that scan's bit for bit.
#include <hip/hip_runtime.h>

#include "common.hpp"
#include "fused.hpp"
#include "merge.hpp"
#include "scan_core.hpp"
#include "select.hpp"

namespace zcgvs_hip {

namespace {

constexpr int kRecoverThreads = kMergeThreads;  // 1024
constexpr int kRecoverChunksPerLane = 8;
constexpr int kRecoverMinLanes = 8;
constexpr int kRecoverListKeys = 4096;  // recoverKernel's running list (32 KB of LDS)
constexpr int kKindI8I8 = 4;

__host__ __device__ constexpr int stagedWordsPerChunk(int kind) {
    // float32 words of one staged 16-byte chunk of the query, or packed words for integer kinds
    return kind == ZCGVS_DTYPE_F32 ? 4 : kind == ZCGVS_DTYPE_F16 ? 8 : kind == ZCGVS_DTYPE_I8 ? 16 : 4;
}

// The selection of list entry `entry` (query q) from the rerun's segments, written like the last
// resort's; false (nothing written) when one of its segments overflowed. Called by the whole
// block.
__device__ bool selectFromRerun(const RecoverArgs& args, int q, int entry, int listed, int batch) {
    __shared__ std::uint32_t lds_hist[kSelectBins];
    __shared__ std::uint32_t lds_scan[kRecoverThreads / kWave];
    __shared__ std::uint64_t lds_keys[kMaxK];
    __shared__ SelectState lds_state;
    __shared__ std::uint32_t lds_over;
    __shared__ std::uint32_t lds_total;
    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const int wave = t / kWave;
    constexpr int kWaves = kRecoverThreads / kWave;
    const int log2 = rerunSegLog2(args.seg_log2, batch, listed);
    const std::uint32_t cap = 1u << log2;
    const int width = args.width;
    if (t == 0) {
        lds_over = 0u;
        lds_total = 0u;
        lds_state.prefix = 0ull;
        lds_state.bits = 0u;
        lds_state.need = static_cast<std::uint32_t>(width);
        lds_state.done = 0u;
        lds_state.count = 0u;
    }
    __syncthreads();
    std::uint32_t own = 0u;
    for (int s = t; s < args.n_seg; s += kRecoverThreads) {
        const std::uint32_t c = args.seg_count[static_cast<std::size_t>(s) * listed + entry];
        if (c > cap) {
            lds_over = 1u;
        }
        own += min(c, cap);
    }
    if (own != 0u) {
        atomicAdd(&lds_total, own);
    }
    __syncthreads();
    if (lds_over != 0u) {
        return false;  // uniform: read after a barrier
    }
    const std::uint32_t total = lds_total;
    // every key of the entry's segments: wavefront w walks segments w, w + 16, ...
    auto forEachKey = [&](auto&& f) {
        for (int s = wave; s < args.n_seg; s += kWaves) {
            const std::uint32_t c = min(args.seg_count[static_cast<std::size_t>(s) * listed + entry], cap);
            const std::uint64_t* src = args.seg + ((static_cast<std::size_t>(s) * listed + entry) << log2);
            for (std::uint32_t j = static_cast<std::uint32_t>(lane); j < c; j += kWave) {
                f(src[j]);
            }
        }
    };
    if (total <= static_cast<std::uint32_t>(width)) {
        if (t == 0) {
            lds_state.done = 1u;
        }
    }
    __syncthreads();
    for (int pass = 0; pass < kSelectPasses && !lds_state.done; ++pass) {
        const int digit = selectDigitWidth(pass);
        for (int i = t; i < (1 << digit); i += kRecoverThreads) {
            lds_hist[i] = 0u;
        }
        __syncthreads();
        const std::uint32_t bits = lds_state.bits;
        const std::uint64_t prefix = lds_state.prefix;
        const int shift = 64 - static_cast<int>(bits) - digit;
        forEachKey([&](std::uint64_t key) {
            if (bits == 0u || (key >> (64 - bits)) == prefix) {
                atomicAdd(&lds_hist[(key >> shift) & ((1u << digit) - 1u)], 1u);
            }
        });
        __syncthreads();
        selectPickBucket<kRecoverThreads>(lds_hist, digit, &lds_state, lds_scan);
    }
    const std::uint64_t cut = total <= static_cast<std::uint32_t>(width) ? 1ull : selectThreshold(lds_state);
    __syncthreads();
    forEachKey([&](std::uint64_t key) {
        if (key >= cut) {
            const std::uint32_t slot = atomicAdd(&lds_state.count, 1u);
            if (slot < static_cast<std::uint32_t>(kMaxK)) {
                lds_keys[slot] = key;
            }
        }
    });
    __syncthreads();
    const std::uint32_t taken = min(min(lds_state.count, static_cast<std::uint32_t>(kMaxK)),
                                    static_cast<std::uint32_t>(width));
    std::uint64_t* dst = args.out_keys + static_cast<std::size_t>(q) * width;
    forEachRanked(lds_keys, taken, [&](std::uint32_t rank, std::uint64_t key) {
        dst[rank] = key;
        if (args.out_index != nullptr) {
            const std::size_t o = static_cast<std::size_t>(q) * width + rank;
            writeHit(key, &args.out_index[o], &args.out_score[o]);
        }
    });
    for (int i = static_cast<int>(taken) + t; i < width; i += kRecoverThreads) {
        dst[i] = 0ull;
        if (args.out_index != nullptr) {
            const std::size_t o = static_cast<std::size_t>(q) * width + i;
            writeHit(0ull, &args.out_index[o], &args.out_score[o]);
        }
    }
    return true;
}

// LDS of the last resort's recomputation: recoverKernel's own, or in mergeRecoverKernel the
// merge's, free once the merge is over.
struct RecomputeLds {
    std::uint32_t* query;  // the staged query: chunks * stagedWordsPerChunk(kind) words
    std::uint32_t* hist;   // kSelectBins
    std::uint32_t* scan;   // kRecoverThreads / kWave
    std::uint64_t* keys;   // kMaxK
    std::uint64_t* list;   // `cap` keys: the running list
    std::uint32_t cap;     // at least kMaxK + kRecoverThreads / 8
    SelectState* state;
    std::uint32_t* fill;   // keys in the list
    std::uint64_t* tau;    // the list's threshold
};

// The last resort for query q, by the whole block: the top-`width` over recomputed scores of the
// whole corpus, written to the outputs. One sweep over the rows in index order keeps every key
// above a running threshold in an LDS list; when the next steps could overfill it, the list is
// cut to its `width` best keys (radix passes over the list, then the keys at or above the cut)
// and the threshold rises to the smallest kept key. The list so always holds the best `width`
// keys of the rows swept so far (keys are unique), and after the sweep the query's exact
// top-`width`. A random corpus appends about width * (1 + ln(n / width)) keys in all; rows that
// ascend in score append every key and cut the list every (cap - width) rows.
template <int kKind, int L>
__device__ __forceinline__ void recomputeQuery(const ScanArgs& scan, const RecoverArgs& args, int chunks, int q,
                                               const RecomputeLds& lds) {
    std::uint32_t* lds_query = lds.query;
    std::uint32_t* lds_hist = lds.hist;
    std::uint32_t* lds_scan = lds.scan;
    std::uint64_t* lds_keys = lds.keys;
    std::uint64_t* lds_list = lds.list;
    SelectState& lds_state = *lds.state;
    std::uint32_t& lds_fill = *lds.fill;
    std::uint64_t& lds_tau = *lds.tau;
    const int t = threadIdx.x;
    const int dim = scan.dim;
    const int width = args.width;
    const long long n = scan.doc_count;
    const int words = chunks * stagedWordsPerChunk(kKind);

    // ---- the query, staged as the VALU scan stages it ----
    if constexpr (kKind == ZCGVS_DTYPE_BINARY) {
        const std::uint32_t* src = static_cast<const std::uint32_t*>(scan.queries) + static_cast<std::size_t>(q) * words;
        for (int i = t; i < words; i += kRecoverThreads) {
            lds_query[i] = src[i];
        }
    } else if constexpr (kKind == kKindI8I8) {
        const std::int8_t* src = static_cast<const std::int8_t*>(scan.queries) + static_cast<std::size_t>(q) * dim;
        for (int w = t; w < words; w += kRecoverThreads) {
            std::uint32_t packed = 0u;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int j = 4 * w + b;
                const int value = j < dim ? static_cast<int>(src[j]) : 0;
                packed |= static_cast<std::uint32_t>(value & 0xFF) << (8 * b);
            }
            lds_query[w] = packed;
        }
    } else {
        const float* src = static_cast<const float*>(scan.queries) + static_cast<std::size_t>(q) * dim;
        float* staged = reinterpret_cast<float*>(lds_query);
        for (int i = t; i < words; i += kRecoverThreads) {
            staged[i] = i < dim ? src[i] : 0.0f;
        }
    }
    if (t == 0) {
        lds_fill = 0u;
        lds_tau = 0ull;
    }
    float inverse = 0.0f;
    if (scan.lexical != nullptr) {
        const float peak = scan.lexical_max[q];
        inverse = peak > 0.0f ? 1.0f / peak : 0.0f;
    }
    const float qscale = scan.query_scales != nullptr ? scan.query_scales[q] : 1.0f;
    __syncthreads();

    const int lane = t & (kWave - 1);
    const int group = lane % L;
    constexpr int kRowsPerPass = kRecoverThreads / L;
    constexpr int kPer = kRecoverChunksPerLane;
    const std::size_t row_bytes = static_cast<std::size_t>(chunks) * 16;
    const std::uint8_t* corpus = static_cast<const std::uint8_t*>(scan.corpus);
    const bool l2 = scan.metric == ZCGVS_METRIC_L2;

    // Key of `row` (valid rows only), identical on the L lanes of the row's group.
    auto keyOf = [&](long long row) -> std::uint64_t {
        const bool masked = scan.mask != nullptr && scan.mask[row] == 0;
        uint4 raw[kPer];
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int c = group + i * L;
            raw[i] = make_uint4(0u, 0u, 0u, 0u);
            if (!masked && c < chunks) {
                raw[i] = loadChunk(corpus + static_cast<std::size_t>(row) * row_bytes + static_cast<std::size_t>(c) * 16);
            }
        }
        float score;
        if constexpr (kKind == ZCGVS_DTYPE_BINARY || kKind == kKindI8I8) {
            int acc = 0;
#pragma unroll
            for (int i = 0; i < kPer; ++i) {
                const int c = group + i * L;
                if (c < chunks) {
                    const uint4 qw = *reinterpret_cast<const uint4*>(lds_query + 4 * c);
                    if constexpr (kKind == ZCGVS_DTYPE_BINARY) {
                        acc += __popc(raw[i].x ^ qw.x) + __popc(raw[i].y ^ qw.y) + __popc(raw[i].z ^ qw.z) +
                               __popc(raw[i].w ^ qw.w);
                    } else {
                        acc = __builtin_amdgcn_sdot4(static_cast<int>(raw[i].x), static_cast<int>(qw.x), acc, false);
                        acc = __builtin_amdgcn_sdot4(static_cast<int>(raw[i].y), static_cast<int>(qw.y), acc, false);
                        acc = __builtin_amdgcn_sdot4(static_cast<int>(raw[i].z), static_cast<int>(qw.z), acc, false);
                        acc = __builtin_amdgcn_sdot4(static_cast<int>(raw[i].w), static_cast<int>(qw.w), acc, false);
                    }
                }
            }
            const int total = groupSum<L>(acc);
            if constexpr (kKind == ZCGVS_DTYPE_BINARY) {
                score = static_cast<float>(dim - 2 * total) / static_cast<float>(dim);
            } else {
                const float row_scale = masked ? 0.0f : scan.row_scales[row];
                const float combined = qscale * row_scale;
                score = static_cast<float>(total) * combined;
            }
        } else {
            using Traits = ChunkTraits<kKind>;
            constexpr int E = Traits::kElems;
            const float* staged = reinterpret_cast<const float*>(lds_query);
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < kPer; ++i) {
                const int c = group + i * L;
                if (c < chunks) {
                    float v[E];
                    Traits::decode(raw[i], scan.scale, v);
                    const float* qv = staged + c * E;
                    if (l2) {
#pragma unroll
                        for (int e = 0; e < E; ++e) {
                            const float d = qv[e] - v[e];
                            acc = fmaf(d, d, acc);
                        }
                    } else {
#pragma unroll
                        for (int e = 0; e < E; ++e) {
                            acc = fmaf(qv[e], v[e], acc);
                        }
                    }
                }
            }
            const float total = groupSum<L>(acc);
            score = l2 ? -total : total;
        }
        float value = masked ? kMaskedScore : score;
        if (scan.lexical != nullptr) {
            const float lex = scan.lexical[static_cast<std::size_t>(q) * n + row];
            value = fuseHybrid(value, lex, scan.dense_weight, inverse);
        }
        return makeKey(value, static_cast<std::uint32_t>(row));
    };

    // Cuts the list's `count` keys (more than width) to its width best at lds_list[0, width) and
    // raises the threshold to the smallest of them. Whole block; ends with a barrier.
    auto cutList = [&](std::uint32_t count) {
        if (t == 0) {
            lds_state.prefix = 0ull;
            lds_state.bits = 0u;
            lds_state.need = static_cast<std::uint32_t>(width);
            lds_state.done = 0u;
            lds_state.count = 0u;
            lds_tau = ~0ull;
        }
        __syncthreads();
        for (int pass = 0; pass < kSelectPasses && !lds_state.done; ++pass) {
            const int digit = selectDigitWidth(pass);
            for (int i = t; i < (1 << digit); i += kRecoverThreads) {
                lds_hist[i] = 0u;
            }
            __syncthreads();
            const std::uint32_t bits = lds_state.bits;
            const std::uint64_t prefix = lds_state.prefix;
            const int shift = 64 - static_cast<int>(bits) - digit;
            for (std::uint32_t i = static_cast<std::uint32_t>(t); i < count; i += kRecoverThreads) {
                const std::uint64_t key = lds_list[i];
                if (bits == 0u || (key >> (64 - bits)) == prefix) {
                    atomicAdd(&lds_hist[(key >> shift) & ((1u << digit) - 1u)], 1u);
                }
            }
            __syncthreads();
            selectPickBucket<kRecoverThreads>(lds_hist, digit, &lds_state, lds_scan);
        }
        // exactly width keys reach the cut (the keys are unique)
        const std::uint64_t cut = selectThreshold(lds_state);
        for (std::uint32_t i = static_cast<std::uint32_t>(t); i < count; i += kRecoverThreads) {
            const std::uint64_t key = lds_list[i];
            if (key >= cut) {
                const std::uint32_t slot = atomicAdd(&lds_state.count, 1u);
                if (slot < static_cast<std::uint32_t>(kMaxK)) {
                    lds_keys[slot] = key;
                }
                atomicMin(&lds_tau, key);
            }
        }
        __syncthreads();
        for (int i = t; i < width; i += kRecoverThreads) {
            lds_list[i] = lds_keys[i];
        }
        if (t == 0) {
            lds_fill = static_cast<std::uint32_t>(width);
        }
        __syncthreads();
    };

    // ---- one sweep in index order, kRowsPerPass rows per step ----
    // A step appends at most kRowsPerPass keys, so a list at most cap - check_every * kRowsPerPass
    // long takes check_every steps before the next check.
    const int check_every = max(1, (static_cast<int>(lds.cap) - width) / kRowsPerPass);
    const std::uint32_t check_limit = lds.cap - static_cast<std::uint32_t>(check_every * kRowsPerPass);
    std::uint64_t tau = 0ull;  // lds_tau, read after each barrier that follows a change
    int step = 0;
    for (long long base = 0; base < n; base += kRowsPerPass) {
        const long long row = base + t / L;
        const bool valid = row < n;
        std::uint64_t key = 0ull;
        if (__any(valid)) {
            key = keyOf(valid ? row : n - 1);
        }
        if (valid && group == 0 && key > tau) {
            lds_list[atomicAdd(&lds_fill, 1u)] = key;
        }
        if (++step == check_every) {
            step = 0;
            __syncthreads();
            const std::uint32_t count = lds_fill;  // uniform: read after the barrier
            if (count > check_limit) {
                cutList(count);
                tau = lds_tau;
            }
        }
    }
    __syncthreads();
    std::uint32_t taken = lds_fill;
    if (taken > static_cast<std::uint32_t>(width)) {
        cutList(taken);
        taken = static_cast<std::uint32_t>(width);
    }

    std::uint64_t* dst = args.out_keys + static_cast<std::size_t>(q) * width;
    forEachRanked(lds_list, taken, [&](std::uint32_t rank, std::uint64_t key) {
        dst[rank] = key;
        if (args.out_index != nullptr) {
            const std::size_t o = static_cast<std::size_t>(q) * width + rank;
            writeHit(key, &args.out_index[o], &args.out_score[o]);
        }
    });
    for (int i = static_cast<int>(taken) + t; i < width; i += kRecoverThreads) {
        dst[i] = 0ull;
        if (args.out_index != nullptr) {
            const std::size_t o = static_cast<std::size_t>(q) * width + i;
            writeHit(0ull, &args.out_index[o], &args.out_score[o]);
        }
    }
}

template <int kKind, int L>
__global__ __launch_bounds__(kRecoverThreads) void recoverKernel(ScanArgs scan, RecoverArgs args,
                                                                 int chunks) {
    extern __shared__ std::uint32_t lds_query[];
    __shared__ std::uint32_t lds_hist[kSelectBins];
    __shared__ std::uint32_t lds_scan[kRecoverThreads / kWave];
    __shared__ std::uint64_t lds_keys[kMaxK];
    __shared__ std::uint64_t lds_list[kRecoverListKeys];
    __shared__ SelectState lds_state;
    __shared__ std::uint32_t lds_fill;
    __shared__ std::uint64_t lds_tau;

    int q = blockIdx.x;
    int entry = 0;
    int listed = 0;
    if (args.force) {
        // every query
    } else if (args.flag_list != nullptr) {
        listed = static_cast<int>(*args.flag_count);
        entry = blockIdx.x;
        if (entry >= listed) {
            return;
        }
        q = static_cast<int>(args.flag_list[entry]);
    } else if (args.flags[q] == 0u) {
        return;
    }
    if (args.seg != nullptr && !args.force && selectFromRerun(args, q, entry, listed, scan.batch)) {
        return;
    }
    recomputeQuery<kKind, L>(scan, args, chunks, q,
                             RecomputeLds{lds_query, lds_hist, lds_scan, lds_keys, lds_list, kRecoverListKeys,
                                          &lds_state, &lds_fill, &lds_tau});
}

// The final merge of a phased search and its exact fallback in one launch: block q merges query
// q's candidates (merge.hpp) and, when that merge flags the query (or with `force`), recomputes
// its selection in the merge's LDS. No separate fallback launch runs for a search without flags.
template <int kKind, int L>
__global__ __launch_bounds__(kRecoverThreads) void mergeRecoverKernel(MergeInputs in, int k, int batch,
                                                                      std::uint64_t* __restrict__ out_keys,
                                                                      std::uint32_t* __restrict__ overflow,
                                                                      int* __restrict__ out_index,
                                                                      float* __restrict__ out_score, ScanArgs scan,
                                                                      RecoverArgs args, int chunks) {
    __shared__ MergeLds lds;
    const int q = static_cast<int>(blockIdx.x);
    const bool flagged = mergeQuery(in, k, batch, out_keys, nullptr, overflow, out_index, out_score, q, lds);
    if (!flagged && !args.force) {
        return;  // uniform
    }
    // the staged query at the end of the candidate LDS, the running list before it
    const std::uint32_t query_keys = (static_cast<std::uint32_t>(chunks * stagedWordsPerChunk(kKind)) + 1u) / 2u;
    const std::uint32_t cap = kSelectLdsKeys - query_keys;
    recomputeQuery<kKind, L>(scan, args, chunks, q,
                             RecomputeLds{reinterpret_cast<std::uint32_t*>(lds.cand + cap), lds.hist, lds.scan,
                                          lds.keys, lds.cand, cap, &lds.state, &lds.valid, &lds.kth});
}

int kindOf(const ScanArgs& scan) {
    if (scan.dtype == ZCGVS_DTYPE_I8 && scan.row_scales != nullptr) {
        return kKindI8I8;
    }
    return scan.dtype;
}

template <int kKind>
int launchKind(int lanes, std::size_t shared, const ScanArgs& scan, const RecoverArgs& args, int chunks,
               hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(scan.batch));
    switch (lanes) {
        case 8: recoverKernel<kKind, 8><<<grid, kRecoverThreads, shared, stream>>>(scan, args, chunks); break;
        case 16: recoverKernel<kKind, 16><<<grid, kRecoverThreads, shared, stream>>>(scan, args, chunks); break;
        case 32: recoverKernel<kKind, 32><<<grid, kRecoverThreads, shared, stream>>>(scan, args, chunks); break;
        default: recoverKernel<kKind, 64><<<grid, kRecoverThreads, shared, stream>>>(scan, args, chunks); break;
    }
    ZCGVS_LAUNCH_CHECK("exact recovery");
    return ZCGVS_OK;
}

template <int kKind>
int launchMergeKind(int lanes, const MergeInputs& in, int k, int batch, std::uint64_t* out_keys,
                    std::uint32_t* overflow, int* out_index, float* out_score, const ScanArgs& scan,
                    const RecoverArgs& args, int chunks, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(batch));
    switch (lanes) {
        case 8:
            mergeRecoverKernel<kKind, 8><<<grid, kRecoverThreads, 0, stream>>>(in, k, batch, out_keys, overflow,
                                                                               out_index, out_score, scan, args, chunks);
            break;
        case 16:
            mergeRecoverKernel<kKind, 16><<<grid, kRecoverThreads, 0, stream>>>(in, k, batch, out_keys, overflow,
                                                                                out_index, out_score, scan, args, chunks);
            break;
        case 32:
            mergeRecoverKernel<kKind, 32><<<grid, kRecoverThreads, 0, stream>>>(in, k, batch, out_keys, overflow,
                                                                                out_index, out_score, scan, args, chunks);
            break;
        default:
            mergeRecoverKernel<kKind, 64><<<grid, kRecoverThreads, 0, stream>>>(in, k, batch, out_keys, overflow,
                                                                                out_index, out_score, scan, args, chunks);
            break;
    }
    ZCGVS_LAUNCH_CHECK("merge and exact recovery");
    return ZCGVS_OK;
}

}  // namespace

bool recoverSupported(const ScanArgs& scan) {
    const std::size_t bytes = rowBytes(scan.dtype, scan.dim);
    if (bytes % 16 != 0 || !aligned16(scan.corpus)) {
        return false;
    }
    const int chunks = static_cast<int>(bytes / 16);
    const int lanes = lanesPerRow(chunks, kRecoverChunksPerLane, kRecoverMinLanes);
    const std::size_t staged = static_cast<std::size_t>(chunks) * stagedWordsPerChunk(kindOf(scan)) * 4;
    return (chunks + lanes - 1) / lanes <= kRecoverChunksPerLane && staged <= 48 * 1024;
}

int launchRecover(const ScanArgs& scan, const RecoverArgs& args, hipStream_t stream) {
    if (args.width <= 0 || args.width > kMaxK || scan.batch <= 0) {
        return setError(ZCGVS_ERR_RUNTIME, "zcgvs recovery: width out of range");
    }
    if (!recoverSupported(scan)) {
        return setError(ZCGVS_ERR_RUNTIME, "zcgvs recovery: row layout not supported");
    }
    const int chunks = static_cast<int>(rowBytes(scan.dtype, scan.dim) / 16);
    const int lanes = lanesPerRow(chunks, kRecoverChunksPerLane, kRecoverMinLanes);
    const int kind = kindOf(scan);
    const std::size_t shared = static_cast<std::size_t>(chunks) * stagedWordsPerChunk(kind) * 4;
    switch (kind) {
        case ZCGVS_DTYPE_F16: return launchKind<ZCGVS_DTYPE_F16>(lanes, shared, scan, args, chunks, stream);
        case ZCGVS_DTYPE_I8: return launchKind<ZCGVS_DTYPE_I8>(lanes, shared, scan, args, chunks, stream);
        case ZCGVS_DTYPE_BINARY: return launchKind<ZCGVS_DTYPE_BINARY>(lanes, shared, scan, args, chunks, stream);
        case kKindI8I8: return launchKind<kKindI8I8>(lanes, shared, scan, args, chunks, stream);
        default: return launchKind<ZCGVS_DTYPE_F32>(lanes, shared, scan, args, chunks, stream);
    }
}

}  // namespace zcgvs_hip

namespace zcgvs_hip {

int launchMergeRecover(const MergeInputs& in, int k, int batch, std::uint64_t* out_keys, std::uint32_t* overflow,
                       int* out_index, float* out_score, const ScanArgs& scan, const RecoverArgs& args,
                       hipStream_t stream) {
    if (args.width != k || k <= 0 || k > kMaxK || batch != scan.batch || batch <= 0 || in.n_seg > kMaxSegments ||
        args.flag_list != nullptr || args.seg != nullptr) {
        return setError(ZCGVS_ERR_RUNTIME, "zcgvs merge and recovery: arguments out of range");
    }
    if (!recoverSupported(scan)) {
        return setError(ZCGVS_ERR_RUNTIME, "zcgvs recovery: row layout not supported");
    }
    const int chunks = static_cast<int>(rowBytes(scan.dtype, scan.dim) / 16);
    const int lanes = lanesPerRow(chunks, kRecoverChunksPerLane, kRecoverMinLanes);
    const int kind = kindOf(scan);
    // the staged query goes to the end of the merge's candidate LDS, before it the running list of
    // at least kMaxK keys and a step's rows
    if (static_cast<std::size_t>(chunks) * stagedWordsPerChunk(kind) * 4 >
        sizeof(MergeLds::cand) - (kMaxK + kRecoverThreads / 8) * sizeof(std::uint64_t)) {
        return setError(ZCGVS_ERR_RUNTIME, "zcgvs merge and recovery: query too large for the merge's LDS");
    }
    switch (kind) {
        case ZCGVS_DTYPE_F16:
            return launchMergeKind<ZCGVS_DTYPE_F16>(lanes, in, k, batch, out_keys, overflow, out_index, out_score, scan,
                                                    args, chunks, stream);
        case ZCGVS_DTYPE_I8:
            return launchMergeKind<ZCGVS_DTYPE_I8>(lanes, in, k, batch, out_keys, overflow, out_index, out_score, scan,
                                                   args, chunks, stream);
        case ZCGVS_DTYPE_BINARY:
            return launchMergeKind<ZCGVS_DTYPE_BINARY>(lanes, in, k, batch, out_keys, overflow, out_index, out_score,
                                                       scan, args, chunks, stream);
        case kKindI8I8:
            return launchMergeKind<kKindI8I8>(lanes, in, k, batch, out_keys, overflow, out_index, out_score, scan,
                                              args, chunks, stream);
        default:
            return launchMergeKind<ZCGVS_DTYPE_F32>(lanes, in, k, batch, out_keys, overflow, out_index, out_score,
                                                    scan, args, chunks, stream);
    }
}

}  // namespace zcgvs_hip
