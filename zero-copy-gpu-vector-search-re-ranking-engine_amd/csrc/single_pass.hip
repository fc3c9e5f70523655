// Single-pass scan for a few queries and a small selection (zcgvs_search_topk with batch <= 4 and
// k or rescore candidates <= a few dozen): one scan launch plus one merge, instead of the phased
// scan's sample, threshold phases and merges between them, whose launches dominate a
// single-query search of a corpus the HBM streams in a hundred microseconds.
//
// Each workgroup (1024 threads, one per compute unit) streams every W-th step of 1024 / L rows
// (W workgroups, L lanes per row) and keeps, per query, every key above its own running
// threshold in an LDS list. When a list could
// overflow before the next check, the workgroup selects its `width` best keys by radix passes over
// the list (select.hpp) and raises the threshold to the smallest of them, so the list is exact:
// it always holds the workgroup's true top-`width`. At the end each workgroup writes its
// top-`width` to its candidate segment, and the per-query merge (topk.hip) selects the global
// top-`width` from the segments. Nothing can overflow, so no fallback pass follows.
//
// Rows are read and scored as the VALU scan and the exact fallback read them (the same lane
// groups of L lanes and up to 8 16-byte chunks per lane, scan_core.hpp), so scores equal theirs
// bit for bit.
#include <hip/hip_runtime.h>

#include "common.hpp"
#include "fused.hpp"
#include "scan_core.hpp"
#include "select.hpp"

namespace zcgvs_hip {

namespace {

constexpr int kSpThreads = 1024;
constexpr int kSpChunksPerLane = 8;  // with 8 lanes at least: the VALU scan's row layout
constexpr int kSpMinLanes = 8;
constexpr int kSpCap = 1024;  // LDS keys per query (one per thread for the compaction)
constexpr int kSpWidthLimit = 32;
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

template <int kKind, int L>
__global__ __launch_bounds__(kSpThreads) void singlePassScanKernel(ScanArgs scan, SinglePassArgs args,
                                                                   int chunks) {
    extern __shared__ std::uint32_t lds_query[];
    __shared__ std::uint64_t lds_keys[kSinglePassQueries][kSpCap];
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

    // Keeps the `width` best keys of query q's list (every thread calls it; q is uniform) and
    // sets the list's threshold to the smallest of them.
    auto compact = [&](int q) __attribute__((always_inline)) {
        const std::uint32_t count = lds_count[q];
        if (count <= static_cast<std::uint32_t>(width)) {
            return;  // (uniform: read after a barrier)
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
            if (static_cast<std::uint32_t>(t) < count) {
                const std::uint64_t key = lds_keys[q][t];
                if (bits == 0u || (key >> (64 - bits)) == prefix) {
                    atomicAdd(&lds_hist[(key >> shift) & ((1u << digit) - 1u)], 1u);
                }
            }
            __syncthreads();
            selectPickBucket<kSpThreads>(lds_hist, digit, &lds_state, lds_scan);
        }
        __syncthreads();
        const std::uint64_t cut = selectThreshold(lds_state);
        const std::uint64_t mine = static_cast<std::uint32_t>(t) < count ? lds_keys[q][t] : 0ull;
        __syncthreads();
        if (t == 0) {
            lds_count[q] = 0u;
        }
        __syncthreads();
        const bool keep = mine != 0ull && mine >= cut;
        if (keep) {
            const std::uint32_t slot = atomicAdd(&lds_count[q], 1u);
            lds_keys[q][slot] = mine;
        }
        // the new threshold: the smallest kept key (exactly the width-th best so far)
        std::uint64_t lo = keep ? mine : ~0ull;
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
        }
        __syncthreads();
    };

    const int lane = t & (kWave - 1);
    const int group = lane % L;
    constexpr int kRowsPerStep = kSpThreads / L;
    constexpr int kPer = kSpChunksPerLane;
    // steps between capacity checks: every list takes at most kRowsPerStep keys per step
    constexpr int kCheckEvery = (kSpCap - kSpWidthLimit) / kRowsPerStep;
    static_assert(kCheckEvery >= 1, "an LDS list holds at least one step of keys beyond the width");
    const std::size_t row_bytes = static_cast<std::size_t>(chunks) * 16;
    const std::uint8_t* corpus = static_cast<const std::uint8_t*>(scan.corpus);
    const bool l2 = scan.metric == ZCGVS_METRIC_L2;
    // Steps interleave over the workgroups (workgroup b takes steps b, b + W, ...), so the
    // workgroups stream neighbouring rows at any moment.
    const long long begin = static_cast<long long>(blockIdx.x) * kRowsPerStep;
    const long long stride = static_cast<long long>(gridDim.x) * kRowsPerStep;
    const long long end = n;

    // this lane's chunks of its row in the step starting at `base` (rows past the corpus and
    // masked rows are not read)
    auto loadStep = [&](long long base, uint4 (&raw)[kPer]) __attribute__((always_inline)) {
        const long long row = base + t / L;
        const long long r = row < end ? row : end - 1;
        const bool skip = row >= end || (scan.mask != nullptr && scan.mask[r] == 0);
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int c = group + i * L;
            raw[i] = make_uint4(0u, 0u, 0u, 0u);
            if (!skip && c < chunks) {
                raw[i] = loadChunkStreaming(corpus + static_cast<std::size_t>(r) * row_bytes + static_cast<std::size_t>(c) * 16);
            }
        }
    };
    // scores of the step's rows against every query, keys above each list's threshold appended
    auto scoreStep = [&](long long base, const uint4 (&raw)[kPer]) __attribute__((always_inline)) {
        const long long row = base + t / L;
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
                for (int i = 0; i < kPer; ++i) {
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
                for (int i = 0; i < kPer; ++i) {
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
                    if (slot < static_cast<std::uint32_t>(kSpCap)) {  // (always: checked between steps)
                        lds_keys[q][slot] = key;
                    }
                }
            }
        }
    };
    // Every kCheckEvery steps: the lists' counts after every wavefront's appends, read between two
    // LDS-only barriers (so the next step's loads stay in flight, and no wavefront appends again
    // before all have read the same counts), and a compaction of any list that the next
    // kCheckEvery steps could overflow.
    int step = 0;
    auto check = [&]() __attribute__((always_inline)) {
        if (++step < kCheckEvery) {
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
            if (counts[q] > static_cast<std::uint32_t>(kSpCap - kCheckEvery * kRowsPerStep)) {
                compact(q);
            }
        }
    };

    uint4 raw[kPer];
    for (long long base = begin; base < end; base += stride) {
        loadStep(base, raw);
        scoreStep(base, raw);
        check();
    }
    __syncthreads();
    for (int q = 0; q < q_count; ++q) {
        compact(q);
    }
    __syncthreads();
    // this workgroup's top-`width` of every query -> its candidate segment
    for (int q = 0; q < q_count; ++q) {
        const std::uint32_t count = min(lds_count[q], static_cast<std::uint32_t>(width));
        const std::size_t seg_row = (static_cast<std::size_t>(blockIdx.x) * q_count + q) << args.seg_log2;
        for (std::uint32_t i = static_cast<std::uint32_t>(t); i < count; i += kSpThreads) {
            args.seg[seg_row + i] = lds_keys[q][i];
        }
        if (t == 0) {
            args.seg_count[static_cast<std::size_t>(blockIdx.x) * q_count + q] = count;
        }
    }
}

template <int kKind>
int launchKind(int lanes, int workgroups, std::size_t shared, const ScanArgs& scan, const SinglePassArgs& args,
               int chunks, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(workgroups));
    switch (lanes) {
        case 8: singlePassScanKernel<kKind, 8><<<grid, kSpThreads, shared, stream>>>(scan, args, chunks); break;
        case 16: singlePassScanKernel<kKind, 16><<<grid, kSpThreads, shared, stream>>>(scan, args, chunks); break;
        case 32: singlePassScanKernel<kKind, 32><<<grid, kSpThreads, shared, stream>>>(scan, args, chunks); break;
        default: singlePassScanKernel<kKind, 64><<<grid, kSpThreads, shared, stream>>>(scan, args, chunks); break;
    }
    ZCGVS_LAUNCH_CHECK("single-pass scan");
    return ZCGVS_OK;
}

}  // namespace

int singlePassWorkgroups() { return deviceComputeUnits(); }

bool singlePassSupported(const ScanArgs& scan, int width) {
    if (scan.batch < 1 || scan.batch > kSinglePassQueries || width < 1 || width > kSpWidthLimit) {
        return false;
    }
    // the merge gathers every workgroup's top-`width` in LDS
    if (static_cast<long long>(singlePassWorkgroups()) * width > kSinglePassMergeKeys) {
        return false;
    }
    const std::size_t bytes = rowBytes(scan.dtype, scan.dim);
    if (bytes % 16 != 0 || !aligned16(scan.corpus)) {
        return false;
    }
    const int chunks = static_cast<int>(bytes / 16);
    const int lanes = lanesPerRow(chunks, kSpChunksPerLane, kSpMinLanes);
    const std::size_t staged = static_cast<std::size_t>(scan.batch) * chunks * spWordsPerChunk(spKindOf(scan)) * 4;
    return (chunks + lanes - 1) / lanes <= kSpChunksPerLane && staged <= kSpQueryLds;
}

int launchSinglePass(const ScanArgs& scan, const SinglePassArgs& args, hipStream_t stream) {
    if (!singlePassSupported(scan, args.width)) {
        return setError(ZCGVS_ERR_RUNTIME, "zcgvs single-pass scan: shape not supported");
    }
    const int chunks = static_cast<int>(rowBytes(scan.dtype, scan.dim) / 16);
    const int lanes = lanesPerRow(chunks, kSpChunksPerLane, kSpMinLanes);
    const int kind = spKindOf(scan);
    const std::size_t shared = static_cast<std::size_t>(scan.batch) * chunks * spWordsPerChunk(kind) * 4;
    const int workgroups = args.workgroups;
    switch (kind) {
        case ZCGVS_DTYPE_F16: return launchKind<ZCGVS_DTYPE_F16>(lanes, workgroups, shared, scan, args, chunks, stream);
        case ZCGVS_DTYPE_I8: return launchKind<ZCGVS_DTYPE_I8>(lanes, workgroups, shared, scan, args, chunks, stream);
        case ZCGVS_DTYPE_BINARY: return launchKind<ZCGVS_DTYPE_BINARY>(lanes, workgroups, shared, scan, args, chunks, stream);
        case kKindI8I8: return launchKind<kKindI8I8>(lanes, workgroups, shared, scan, args, chunks, stream);
        default: return launchKind<ZCGVS_DTYPE_F32>(lanes, workgroups, shared, scan, args, chunks, stream);
    }
}

}  // namespace zcgvs_hip
