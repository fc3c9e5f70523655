// Single-pass scan for a few queries (zcgvs_search_topk with batch <= 4 and k or rescore
// candidates up to 1024): one scan launch plus one or two merges, instead of the phased scan's
// sample, threshold phases and merges between them, whose launches dominate a single-query search
// of a corpus the HBM streams in a hundred microseconds.
//
// Each workgroup (1024 threads, one per compute unit) streams every W-th step of 1024 / L rows
// (W workgroups, L lanes per row) and keeps, per query, every key above its own running
// threshold in an LDS list. When a list could
// overflow before the next check, the workgroup selects its `width` best keys by radix passes over
// the list (select.hpp), or by ranking every key when the list holds at most 256, and raises the
// threshold to the smallest of them, so the list is exact:
// it always holds the workgroup's true top-`width`. At the end each workgroup writes its
// top-`width` to its candidate segment (sorted descending when width <= 256), and the per-query
// merge (topk.hip) selects the global top-`width` from the segments: for width <= 32 from the
// segments whose first key reaches the width-th best first key, for wide selections after
// merging groups of workgroups first. A
// list holds max(1024, 4 * width) keys for a narrow selection and the query's whole share of the
// list LDS for a wide one (less when four queries share the LDS), so compactions are rare.
// Nothing can overflow, so no fallback pass follows.
//
// Rows are read and scored as the VALU scan and the exact fallback read them (the same lane
// groups of L lanes and up to 8 16-byte chunks per lane, scan_core.hpp), so scores equal theirs
// bit for bit.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.hpp"
#include "fused.hpp"
#include "scan_core.hpp"
#include "select.hpp"

namespace zcgvs_hip {

namespace {

constexpr int kSpThreads = 1024;
constexpr int kSpChunksPerLane = 8;  // with 8 lanes at least: the VALU scan's row layout
constexpr int kSpMinLanes = 8;
constexpr int kSpListKeys = 12288;  // LDS keys of all queries' lists together (96 KB)
constexpr int kSpMinCap = 1024;     // keys per query list at least
constexpr int kSpRankKeys = 256;    // lists up to this long are compacted by ranking, not radix passes
constexpr int kKindI8I8 = 4;
constexpr std::size_t kSpQueryLds = 32 * 1024;

__host__ __device__ constexpr int spWordsPerChunk(int kind) {
    return kind == ZCGVS_DTYPE_F32 ? 4 : kind == ZCGVS_DTYPE_F16 ? 8 : kind == ZCGVS_DTYPE_I8 ? 16 : 4;
}

int spKindOf(const ScanArgs& scan) {
    if (scan.dtype == ZCGVS_DTYPE_I8 && scan.row_scales != nullptr) {
        return kKindI8I8;
    }
    return scan.dtype;
}

// A workgroup barrier that waits only for this wavefront's LDS operations, not its global loads.
__device__ inline void ldsBarrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt not waited on
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int kKind, int L, int kSets>
__global__ __launch_bounds__(kSpThreads) void singlePassScanKernel(ScanArgs scan, SinglePassArgs args,
                                                                   int chunks) {
    extern __shared__ std::uint32_t lds_query[];
    __shared__ std::uint64_t lds_keys[kSpListKeys];  // query q's list at q * cap
    __shared__ std::uint32_t lds_count[kSinglePassQueries];
    __shared__ std::uint64_t lds_tau[kSinglePassQueries];
    __shared__ std::uint32_t lds_hist[kSelectBins];
    __shared__ std::uint32_t lds_scan[kSpThreads / kWave];
    __shared__ std::uint64_t lds_wave_lo[kSpThreads / kWave];
    __shared__ SelectState lds_state;

    const int t = threadIdx.x;
    const int dim = scan.dim;
    const int q_count = scan.batch;  // <= kSinglePassQueries
    const int width = args.width;
    const long long n = scan.doc_count;
    const int words = chunks * spWordsPerChunk(kKind);

    const int cap = args.cap;  // keys per query list (width + at least one check's appends)
    const int lane = t & (kWave - 1);
    const int group = lane % L;
    // A step: kSets row sets of kSpThreads / L consecutive rows; a lane reads kPerRow chunks of
    // its row in every set (several sets for short rows, so each lane keeps up to
    // kSpChunksPerLane chunks in flight).
    constexpr int kGroupsPerSet = kSpThreads / L;
    constexpr int kRowsPerStep = kGroupsPerSet * kSets;
    constexpr int kPer = kSpChunksPerLane;
    constexpr int kPerRow = kPer / kSets;
    static_assert(kPerRow * kSets == kPer, "row sets split the lane's chunks evenly");
    // steps between capacity checks: every list takes at most kRowsPerStep keys per step (the
    // host makes cap - width at least one step's rows). A narrow selection checks as often as its
    // list allows, so the list stays short and its compactions are rankings; a wide one (more
    // than kSpRankKeys keys, compacted by radix passes) checks half as often, so a list is cut
    // only once it is about half full.
    const int check_every = width > kSpRankKeys ? max(1, (cap - width) / (2 * kRowsPerStep))
                                                : (cap - width) / kRowsPerStep;
    const std::size_t row_bytes = static_cast<std::size_t>(chunks) * 16;
    const std::uint8_t* corpus = static_cast<const std::uint8_t*>(scan.corpus);
    const bool l2 = scan.metric == ZCGVS_METRIC_L2;
    // Steps interleave over the workgroups (workgroup b takes steps b, b + W, ...), so the
    // workgroups stream neighbouring rows at any moment.
    const long long begin = static_cast<long long>(blockIdx.x) * kRowsPerStep;
    const long long stride = static_cast<long long>(gridDim.x) * kRowsPerStep;
    const long long end = n;

    // this lane's chunks of its rows in the step starting at `base` (rows past the corpus and
    // masked rows are not read)
    auto loadStep = [&](long long base, uint4 (&raw)[kPer]) __attribute__((always_inline)) {
#pragma unroll
        for (int set = 0; set < kSets; ++set) {
            const long long row = base + set * kGroupsPerSet + t / L;
            const long long r = row < end ? row : end - 1;
            const bool skip = row >= end || (scan.mask != nullptr && scan.mask[r] == 0);
#pragma unroll
            for (int i = 0; i < kPerRow; ++i) {
                const int c = group + i * L;
                uint4& chunk = raw[set * kPerRow + i];
                chunk = make_uint4(0u, 0u, 0u, 0u);
                if (!skip && c < chunks) {
                    chunk = loadChunkStreaming(corpus + static_cast<std::size_t>(r) * row_bytes + static_cast<std::size_t>(c) * 16);
                }
            }
        }
    };
    // The first step's loads go out before the queries are staged, so the two round trips overlap.
    uint4 raw[kPer];
    if (begin < end) {
        loadStep(begin, raw);
    }

    // ---- the queries, staged as the VALU scan stages them ----
    for (int q = 0; q < q_count; ++q) {
        std::uint32_t* staged = lds_query + q * words;
        if constexpr (kKind == ZCGVS_DTYPE_BINARY) {
            const std::uint32_t* src = static_cast<const std::uint32_t*>(scan.queries) + static_cast<std::size_t>(q) * words;
            for (int i = t; i < words; i += kSpThreads) {
                staged[i] = src[i];
            }
        } else if constexpr (kKind == kKindI8I8) {
            const std::int8_t* src = static_cast<const std::int8_t*>(scan.queries) + static_cast<std::size_t>(q) * dim;
            for (int w = t; w < words; w += kSpThreads) {
                std::uint32_t packed = 0u;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const int j = 4 * w + b;
                    const int value = j < dim ? static_cast<int>(src[j]) : 0;
                    packed |= static_cast<std::uint32_t>(value & 0xFF) << (8 * b);
                }
                staged[w] = packed;
            }
        } else {
            const float* src = static_cast<const float*>(scan.queries) + static_cast<std::size_t>(q) * dim;
            float* fstaged = reinterpret_cast<float*>(staged);
            for (int i = t; i < words; i += kSpThreads) {
                fstaged[i] = i < dim ? src[i] : 0.0f;
            }
        }
    }
    if (t < kSinglePassQueries) {
        lds_count[t] = 0u;
        lds_tau[t] = 0ull;
    }
    float inverse[kSinglePassQueries];
    float qscale[kSinglePassQueries];
#pragma unroll
    for (int q = 0; q < kSinglePassQueries; ++q) {
        inverse[q] = 0.0f;
        qscale[q] = 1.0f;
        if (q < q_count) {
            if (scan.lexical != nullptr) {
                const float peak = scan.lexical_max[q];
                inverse[q] = peak > 0.0f ? 1.0f / peak : 0.0f;
            }
            if (scan.query_scales != nullptr) {
                qscale[q] = scan.query_scales[q];
            }
        }
    }
    __syncthreads();

    // Keeps the best min(count, width) of query q's `count` list keys (2 <= count <= kSpRankKeys),
    // sorted descending at the front of the list: every key's rank (the number of keys above it;
    // all keys are unique) from `parts` threads per key whose counts meet in LDS, then the kept
    // keys move to their ranks. Four barriers instead of the radix passes' dozens.
    auto rankKeep = [&](int q, std::uint32_t count) __attribute__((always_inline)) {
        std::uint64_t* list = lds_keys + q * cap;
        std::uint32_t* rank_of = lds_hist;
        for (std::uint32_t i = static_cast<std::uint32_t>(t); i < count; i += kSpThreads) {
            rank_of[i] = 0u;
        }
        __syncthreads();
        const std::uint32_t parts = static_cast<std::uint32_t>(kSpThreads) / count;
        const std::uint32_t per = (count + parts - 1u) / parts;
        if (static_cast<std::uint32_t>(t) < count * parts) {
            const std::uint32_t i = static_cast<std::uint32_t>(t) / parts;
            const std::uint32_t j0 = (static_cast<std::uint32_t>(t) - i * parts) * per;
            const std::uint32_t j1 = min(count, j0 + per);
            const std::uint64_t key = list[i];
            std::uint32_t above = 0u;
            for (std::uint32_t j = j0; j < j1; ++j) {
                above += list[j] > key ? 1u : 0u;
            }
            if (above != 0u) {
                atomicAdd(&rank_of[i], above);
            }
        }
        __syncthreads();
        std::uint64_t key = 0ull;
        std::uint32_t rank = ~0u;
        if (static_cast<std::uint32_t>(t) < count) {
            key = list[t];
            rank = rank_of[t];
        }
        __syncthreads();  // every key read before any moves
        if (rank < static_cast<std::uint32_t>(width)) {
            list[rank] = key;
            if (rank == static_cast<std::uint32_t>(width) - 1u) {
                lds_tau[q] = key;
            }
        }
        if (t == 0) {
            lds_count[q] = min(count, static_cast<std::uint32_t>(width));
        }
        __syncthreads();
    };
    // Keeps the `width` best keys of query q's list (every thread calls it; q is uniform) and
    // sets the list's threshold to the smallest of them.
    auto compact = [&](int q) __attribute__((always_inline)) {
        std::uint64_t* list = lds_keys + q * cap;
        const std::uint32_t count = lds_count[q];
        if (count <= static_cast<std::uint32_t>(width)) {
            return;  // (uniform: read after a barrier)
        }
        if (count <= static_cast<std::uint32_t>(kSpRankKeys)) {
            rankKeep(q, count);
            return;
        }
        if (t == 0) {
            lds_state.prefix = 0ull;
            lds_state.bits = 0u;
            lds_state.need = static_cast<std::uint32_t>(width);
            lds_state.done = 0u;
        }
        for (int pass = 0; pass < kSelectPasses; ++pass) {
            const int digit = selectDigitWidth(pass);
            for (int i = t; i < (1 << digit); i += kSpThreads) {
                lds_hist[i] = 0u;
            }
            __syncthreads();
            if (lds_state.done) {
                break;
            }
            const std::uint32_t bits = lds_state.bits;
            const std::uint64_t prefix = lds_state.prefix;
            const int shift = 64 - static_cast<int>(bits) - digit;
            for (std::uint32_t i = static_cast<std::uint32_t>(t); i < count; i += kSpThreads) {
                const std::uint64_t key = list[i];
                if (bits == 0u || (key >> (64 - bits)) == prefix) {
                    atomicAdd(&lds_hist[(key >> shift) & ((1u << digit) - 1u)], 1u);
                }
            }
            __syncthreads();
            selectPickBucket<kSpThreads>(lds_hist, digit, &lds_state, lds_scan);
        }
        __syncthreads();
        const std::uint64_t cut = selectThreshold(lds_state);
        // In place, 1024 keys a round: a kept key moves to a position no later than its own, and
        // every key of a round is read before any of the round's moves, so nothing unread is
        // overwritten. lds_state.count is the number of keys kept so far.
        if (t == 0) {
            lds_state.count = 0u;
        }
        std::uint64_t lo = ~0ull;
        for (std::uint32_t base = 0; base < count; base += kSpThreads) {
            const std::uint32_t i = base + static_cast<std::uint32_t>(t);
            const std::uint64_t key = i < count ? list[i] : 0ull;
            const bool keep = key != 0ull && key >= cut;
            __syncthreads();  // the round's reads (and the last round's count) before its moves
            const std::uint64_t mask = __builtin_amdgcn_ballot_w64(keep);
            const std::uint32_t before = __builtin_amdgcn_mbcnt_hi(static_cast<std::uint32_t>(mask >> 32),
                                                                   __builtin_amdgcn_mbcnt_lo(static_cast<std::uint32_t>(mask), 0u));
            if ((t & (kWave - 1)) == 0) {
                lds_scan[t / kWave] = static_cast<std::uint32_t>(__builtin_popcountll(mask));
            }
            __syncthreads();
            std::uint32_t offset = lds_state.count;
            for (int w = 0; w < t / kWave; ++w) {
                offset += lds_scan[w];
            }
            if (keep) {
                list[offset + before] = key;
                lo = min(lo, key);
            }
            __syncthreads();  // every wavefront has read lds_state.count and lds_scan
            if (t == kSpThreads - 1) {
                std::uint32_t round = 0u;
                for (int w = 0; w < kSpThreads / kWave; ++w) {
                    round += lds_scan[w];
                }
                lds_state.count += round;
            }
        }
        // the new threshold: the smallest kept key (exactly the width-th best so far)
        lo = waveReduce64(lo, [](std::uint64_t a, std::uint64_t b) { return min(a, b); });
        if ((t & (kWave - 1)) == 0) {
            lds_wave_lo[t / kWave] = lo;
        }
        __syncthreads();
        if (t == 0) {
            std::uint64_t all = ~0ull;
            for (int w = 0; w < kSpThreads / kWave; ++w) {
                all = min(all, lds_wave_lo[w]);
            }
            lds_tau[q] = all;
            lds_count[q] = lds_state.count;
        }
        __syncthreads();
    };

    // scores of the step's rows against every query, keys above each list's threshold appended
    auto scoreStep = [&](long long base, const uint4 (&raw_step)[kPer]) __attribute__((always_inline)) {
#pragma unroll
        for (int set = 0; set < kSets; ++set) {
            const uint4* raw = raw_step + set * kPerRow;
            const long long row = base + set * kGroupsPerSet + t / L;
            const bool valid = row < end;
            const long long r = valid ? row : end - 1;
            const bool masked = scan.mask != nullptr && scan.mask[r] == 0;
            float row_scale = 1.0f;
            if constexpr (kKind == kKindI8I8) {
                row_scale = masked ? 0.0f : scan.row_scales[r];
            }
#pragma unroll
            for (int q = 0; q < kSinglePassQueries; ++q) {
                if (q >= q_count) {
                    break;
                }
                const std::uint32_t* staged = lds_query + q * words;
                float score;
                if constexpr (kKind == ZCGVS_DTYPE_BINARY || kKind == kKindI8I8) {
                    int acc = 0;
#pragma unroll
                    for (int i = 0; i < kPerRow; ++i) {
                        const int c = group + i * L;
                        if (c < chunks) {
                            const uint4 qw = *reinterpret_cast<const uint4*>(staged + 4 * c);
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
                        const float combined = qscale[q] * row_scale;
                        score = static_cast<float>(total) * combined;
                    }
                } else {
                    using Traits = ChunkTraits<kKind>;
                    constexpr int E = Traits::kElems;
                    const float* fstaged = reinterpret_cast<const float*>(staged);
                    float acc = 0.0f;
#pragma unroll
                    for (int i = 0; i < kPerRow; ++i) {
                        const int c = group + i * L;
                        if (c < chunks) {
                            float v[E];
                            Traits::decode(raw[i], scan.scale, v);
                            const float* qv = fstaged + c * E;
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
                if (valid && group == 0) {
                    float value = masked ? kMaskedScore : score;
                    if (scan.lexical != nullptr) {
                        const float lex = scan.lexical[static_cast<std::size_t>(q) * n + row];
                        value = fuseHybrid(value, lex, scan.dense_weight, inverse[q]);
                    }
                    const std::uint64_t key = makeKey(value, static_cast<std::uint32_t>(row));
                    if (key > lds_tau[q]) {
                        const std::uint32_t slot = atomicAdd(&lds_count[q], 1u);
                        if (slot < static_cast<std::uint32_t>(cap)) {  // (always: checked between steps)
                            lds_keys[q * cap + slot] = key;
                        }
                    }
                }
            }
        }
    };

    // Every check_every steps: the lists' counts after every wavefront's appends, read between two
    // LDS-only barriers (so the next step's loads stay in flight, and no wavefront appends again
    // before all have read the same counts), and a compaction of any list that the next
    // check_every steps could overflow.
    int step = 0;
    auto check = [&]() __attribute__((always_inline)) {
        if (++step < check_every) {
            return;
        }
        step = 0;
        ldsBarrier();
        std::uint32_t counts[kSinglePassQueries];
#pragma unroll
        for (int q = 0; q < kSinglePassQueries; ++q) {
            counts[q] = q < q_count ? lds_count[q] : 0u;
        }
        ldsBarrier();
#pragma unroll
        for (int q = 0; q < kSinglePassQueries; ++q) {
            if (counts[q] > static_cast<std::uint32_t>(cap - check_every * kRowsPerStep)) {
                compact(q);
            }
        }
    };

    for (long long base = begin; base < end; base += stride) {
        scoreStep(base, raw);
        check();
        if (base + stride < end) {
            loadStep(base + stride, raw);
        }
    }
    __syncthreads();
    // The final lists: each workgroup's top-`width`, sorted descending when width <= kSpRankKeys
    // (the merge of narrow selections relies on it).
    for (int q = 0; q < q_count; ++q) {
        const std::uint32_t before = lds_count[q];
        compact(q);
        const bool ranked = before > static_cast<std::uint32_t>(width) && before <= static_cast<std::uint32_t>(kSpRankKeys);
        const std::uint32_t count = lds_count[q];  // (uniform: compact ends with a barrier)
        if (width <= kSpRankKeys && !ranked && count >= 2u) {
            rankKeep(q, count);  // a list compact left as it was, or compacted by radix passes
        }
    }
    __syncthreads();
    // This workgroup's top-`width` of every query -> its candidate segment. With G merge groups
    // workgroup b belongs to group g = b % G as its segment s = b / G, and the list of query q
    // goes to the segment of (s, q * G + g) in a layout of q_count * G merge queries, so the first
    // merge treats every (query, group) pair as a query of its own.
    const int groups = args.groups;
    const int g = static_cast<int>(blockIdx.x) % groups;
    const std::size_t s_index = blockIdx.x / groups;
    for (int q = 0; q < q_count; ++q) {
        const std::uint32_t count = min(lds_count[q], static_cast<std::uint32_t>(width));
        const std::size_t merge_q = static_cast<std::size_t>(q) * groups + g;
        const std::size_t slot = s_index * static_cast<std::size_t>(q_count * groups) + merge_q;
        for (std::uint32_t i = static_cast<std::uint32_t>(t); i < count; i += kSpThreads) {
            args.seg[(slot << args.seg_log2) + i] = lds_keys[q * cap + i];
        }
        if (t == 0) {
            args.seg_count[slot] = count;
        }
    }
}

// Lanes per row and row sets per step for rows of `chunks` 16-byte chunks: the VALU scan's lane
// count (at least 8 lanes, at most 8 chunks a lane); rows that leave a lane's 8 chunks mostly
// unused (at most 4 chunks a lane) take several rows per step, up to L sets.
struct SpLayout {
    int lanes = 0;
    int sets = 1;
};

SpLayout spLayout(int chunks) {
    SpLayout layout;
    layout.lanes = lanesPerRow(chunks, kSpChunksPerLane, kSpMinLanes);
    int per_row = 1;
    while (per_row * layout.lanes < chunks) {
        per_row *= 2;
    }
    layout.sets = std::min(kSpChunksPerLane / per_row, layout.lanes);
    return layout;
}

template <int kKind, int L, int kSets>
int launchSets(int workgroups, std::size_t shared, const ScanArgs& scan, const SinglePassArgs& args, int chunks,
               hipStream_t stream) {
    singlePassScanKernel<kKind, L, kSets><<<dim3(static_cast<unsigned>(workgroups)), kSpThreads, shared, stream>>>(
        scan, args, chunks);
    ZCGVS_LAUNCH_CHECK("single-pass scan");
    return ZCGVS_OK;
}

template <int kKind>
int launchKind(const SpLayout& layout, int workgroups, std::size_t shared, const ScanArgs& scan,
               const SinglePassArgs& args, int chunks, hipStream_t stream) {
    switch (layout.lanes * 16 + layout.sets) {
        case 1 * 16 + 1: return launchSets<kKind, 1, 1>(workgroups, shared, scan, args, chunks, stream);
        case 2 * 16 + 2: return launchSets<kKind, 2, 2>(workgroups, shared, scan, args, chunks, stream);
        case 4 * 16 + 4: return launchSets<kKind, 4, 4>(workgroups, shared, scan, args, chunks, stream);
        case 8 * 16 + 8: return launchSets<kKind, 8, 8>(workgroups, shared, scan, args, chunks, stream);
        case 8 * 16 + 4: return launchSets<kKind, 8, 4>(workgroups, shared, scan, args, chunks, stream);
        case 8 * 16 + 2: return launchSets<kKind, 8, 2>(workgroups, shared, scan, args, chunks, stream);
        case 8 * 16 + 1: return launchSets<kKind, 8, 1>(workgroups, shared, scan, args, chunks, stream);
        case 16 * 16 + 1: return launchSets<kKind, 16, 1>(workgroups, shared, scan, args, chunks, stream);
        case 32 * 16 + 1: return launchSets<kKind, 32, 1>(workgroups, shared, scan, args, chunks, stream);
        case 64 * 16 + 1: return launchSets<kKind, 64, 1>(workgroups, shared, scan, args, chunks, stream);
        default: return setError(ZCGVS_ERR_RUNTIME, "zcgvs single-pass scan: no kernel for this row layout");
    }
}

}  // namespace

SinglePassShape singlePassShape(const ScanArgs& scan, int width) {
    SinglePassShape shape;
    if (scan.batch < 1 || scan.batch > kSinglePassQueries || width < 1 || width > kMaxK) {
        return shape;
    }
    const std::size_t bytes = rowBytes(scan.dtype, scan.dim);
    if (bytes % 16 != 0 || !aligned16(scan.corpus)) {
        return shape;
    }
    const int chunks = static_cast<int>(bytes / 16);
    const SpLayout layout = spLayout(chunks);
    const std::size_t staged = static_cast<std::size_t>(scan.batch) * chunks * spWordsPerChunk(spKindOf(scan)) * 4;
    if ((chunks + layout.lanes - 1) / layout.lanes > kSpChunksPerLane || staged > kSpQueryLds) {
        return shape;
    }
    // A list holds its width best keys plus at least one check's appends (rows per step): for a
    // narrow selection four times the width, or two steps' rows beyond it; a wide one (compacted
    // by radix passes) takes the queries' whole share of the list LDS, so it is cut about once per
    // workgroup (binary 50M x 1024, 1000 keys, one query: 1.013 against 1.04-1.05 ms per scan).
    const int rows_per_step = kSpThreads / layout.lanes * layout.sets;
    const int share = kSpListKeys / scan.batch / 64 * 64;
    const int cap = width > kSpRankKeys
                        ? share
                        : std::min(share,
                                   std::max({kSpMinCap, (4 * width + 63) / 64 * 64, width + 2 * rows_per_step}));
    if (cap - width < rows_per_step) {
        return shape;
    }
    // Merge groups: one merge of every workgroup's list when the lists fit its LDS gather or are
    // sorted and at most kSortedSelectMaxK long (the sorted-segment merge reads only the lists
    // whose first key can reach the result), otherwise groups of workgroups merged first (each
    // group's lists in LDS, at most 8192 keys) and their results merged after.
    const int units = deviceComputeUnits();
    int groups = 1;
    while (width > kSortedSelectMaxK &&
           static_cast<long long>(units / groups) * width > (groups == 1 ? kSinglePassMergeKeys : 8192) &&
           groups < units) {
        groups *= 2;
    }
    shape.supported = true;
    shape.groups = groups;
    shape.workgroups = std::max(groups, units / groups * groups);
    shape.cap = cap;
    int log2 = 0;
    while ((1 << log2) < width) {
        ++log2;
    }
    shape.seg_log2 = log2;
    return shape;
}

bool singlePassSupported(const ScanArgs& scan, int width) { return singlePassShape(scan, width).supported; }

int launchSinglePass(const ScanArgs& scan, const SinglePassArgs& args, hipStream_t stream) {
    const SinglePassShape shape = singlePassShape(scan, args.width);
    if (!shape.supported || args.cap != shape.cap || args.groups != shape.groups ||
        args.workgroups % args.groups != 0) {
        return setError(ZCGVS_ERR_RUNTIME, "zcgvs single-pass scan: shape not supported");
    }
    const int chunks = static_cast<int>(rowBytes(scan.dtype, scan.dim) / 16);
    const SpLayout layout = spLayout(chunks);
    const int kind = spKindOf(scan);
    const std::size_t shared = static_cast<std::size_t>(scan.batch) * chunks * spWordsPerChunk(kind) * 4;
    const int workgroups = args.workgroups;
    switch (kind) {
        case ZCGVS_DTYPE_F16: return launchKind<ZCGVS_DTYPE_F16>(layout, workgroups, shared, scan, args, chunks, stream);
        case ZCGVS_DTYPE_I8: return launchKind<ZCGVS_DTYPE_I8>(layout, workgroups, shared, scan, args, chunks, stream);
        case ZCGVS_DTYPE_BINARY: return launchKind<ZCGVS_DTYPE_BINARY>(layout, workgroups, shared, scan, args, chunks, stream);
        case kKindI8I8: return launchKind<kKindI8I8>(layout, workgroups, shared, scan, args, chunks, stream);
        default: return launchKind<ZCGVS_DTYPE_F32>(layout, workgroups, shared, scan, args, chunks, stream);
    }
}

}  // namespace zcgvs_hip
