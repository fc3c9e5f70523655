// Fused scan-and-filter: the pieces shared by the VALU and MFMA scan kernels of the fused search.
//
// Phases. The corpus is cut into blocks of `block_rows` rows. A phase visits the blocks whose
// index is a multiple of `stride` but (when skip > 0) not a multiple of stride * skip, i.e. the
// phases form a coarse-to-fine interleaved sampling of the whole corpus: phase 0 sees every
// stride_0-th block, phase 1 every stride_1-th block not yet seen, ..., the last phase every
// remaining block. Phase 0 writes every key to a fixed slot ("dense"); later phases keep only
// keys above the per-query threshold, the k-th best key found by the phases before, which is
// a lower bound of the final k-th best key, so no final hit is ever dropped.
//
// Emission. Each workgroup appends its candidates for query q to its own segment
// seg[(s * batch + q) << seg_log2 ...] (s = the workgroup; the int8 MFMA scan gives each workgroup
// two segments, one per row half of a query's lanes, and counts in registers), counting with LDS
// atomics (no global atomics, so the scan's memory pipeline never waits on a returning atomic),
// and stores its per-query counts when it finishes. A count above the segment capacity is
// reported as overflow by the merge.
#pragma once

#include "common.hpp"
#include "select.hpp"

namespace zcgvs_hip {

struct PhaseArgs {
    long long stride = 1;
    long long skip = 0;
    long long items = 0;
    int dense = 0;
    // A sketch phase (int8 MFMA scan, binary streaming scan) emits no keys: each of its slots (2
    // per workgroup in the int8 scan, 8 in the binary one) keeps the best exact score of its rows
    // per query, written to EmitArgs::sketch.
    int sketch = 0;
    // A store phase (with dense set; the launchers' score matrix) writes every valid row's score,
    // as a float, to EmitArgs::scores[q * doc_count + row] instead of a key.
    int store = 0;
    int block_rows = 64;
};

struct EmitArgs {
    const std::uint64_t* tau = nullptr;  // [batch] thresholds (ignored for dense phases)
    std::uint64_t* dense = nullptr;      // [batch, dense_stride]
    long long dense_stride = 0;
    std::uint64_t* seg = nullptr;        // [n_wg, batch, 1 << seg_log2]
    std::uint32_t* seg_count = nullptr;  // [n_wg, batch]
    int seg_log2 = 0;
    float* sketch = nullptr;             // sketch phases: [slots, batch] best score per slot
    float* scores = nullptr;             // store phases: [batch, doc_count] scores
    // Rerun of the exact fallback (int8 MFMA scan, binary streaming scan): only the F = *q_list_count queries
    // q_list[0..F) are scanned. List entry e of query q = q_list[e] owns the segments
    // seg[(s * F + e) << rerunSegLog2(seg_log2, batch, F)] with counts seg_count[s * F + e], so
    // the F queries share the whole segment buffer of the batch.
    const std::uint32_t* q_list = nullptr;
    const std::uint32_t* q_list_count = nullptr;
};

// Slots per (segment, list entry) of a rerun over F of the batch's queries: the batch's capacity
// 2^seg_log2 times the largest power of two <= batch / F (at most 2^23 slots).
__host__ __device__ inline int rerunSegLog2(int seg_log2, int batch, int listed) {
    int shift = 0;
    while (listed > 0 && (static_cast<long long>(listed) << (shift + 1)) <= batch) {
        ++shift;
    }
    return seg_log2 + shift < 23 ? seg_log2 + shift : 23;
}

// First block of work item j of a phase: the j-th multiple of `stride` that is not a multiple
// of stride * skip. Item counts and skips stay below 2^31, so the division is 32-bit.
__device__ __forceinline__ long long phaseBlock(long long j, long long stride, long long skip) {
    if (skip == 0) {
        return j * stride;
    }
    const std::uint32_t j32 = static_cast<std::uint32_t>(j);
    const std::uint32_t visited = j32 + j32 / static_cast<std::uint32_t>(skip - 1) + 1u;
    return static_cast<long long>(visited) * stride;
}

// Work items of a phase over `blocks` blocks.
inline long long phaseItems(long long blocks, long long stride, long long skip) {
    const long long multiples = (blocks + stride - 1) / stride;
    if (skip == 0) {
        return multiples;
    }
    return multiples - (multiples + skip - 1) / skip;
}

// A score floor for the keys above a threshold key `tau`: keys order by their score's ordered bits
// first, so key > tau needs score >= keyScore(tau). The floor holds only when tau is a real key
// whose score is not NaN (NaN scores rank lowest and fail every comparison); *gated is false
// otherwise and every score must then be keyed and compared.
__device__ __forceinline__ float keyFloor(std::uint64_t tau, bool* gated) {
    const float score = keyScore(tau);
    *gated = tau != 0ull && score == score;
    return score;
}

// Appends `key` to query q's segment of this workgroup (lds_count: this workgroup's per-query
// counts for the launch's query range, indexed by q - q_offset).
__device__ __forceinline__ void appendCandidate(const EmitArgs& emit, std::uint32_t* lds_count,
                                                int q, int q_offset, int batch,
                                                std::uint64_t key) {
    const std::uint32_t slot = atomicAdd(&lds_count[q - q_offset], 1u);
    if (slot < (1u << emit.seg_log2)) {
        emit.seg[((static_cast<std::size_t>(blockIdx.x) * batch + q) << emit.seg_log2) + slot] = key;
    }
}

// Hybrid fusion of src/cuda/lexical.cu:67-74 for one (query, row): w * dense + ((1 - w) * lex) *
// inverse, as separate IEEE operations in the reference's operand order.
__device__ __forceinline__ float fuseHybrid(float dense, float lexical, float weight,
                                            float inverse) {
#pragma clang fp contract(off)
    const float a = weight * dense;
    const float b = (1.0f - weight) * lexical;
    const float c = b * inverse;
    return a + c;
}

// ---- internal launch interfaces ------------------------------------------------------------

struct ScanArgs {
    const void* corpus = nullptr;
    long long doc_count = 0;
    int dim = 0;
    int dtype = 0;               // zcgvs_dtype; I8 with row_scales != nullptr = per-vector mode
    float scale = 1.0f;
    const float* row_scales = nullptr;
    // MFMA scan: when set, the last (partial) tile reads its 64 scales here (valid rows, then NaN)
    // and every full tile reads row_scales directly; when null, row_scales is padded to whole
    // tiles.
    const float* tail_scales = nullptr;
    const void* queries = nullptr;  // f32 [batch, dim] | packed words [batch, W] | int8 [batch, dim]
    const float* query_scales = nullptr;
    int batch = 0;
    int metric = 0;
    const std::uint8_t* mask = nullptr;
    const float* lexical = nullptr;      // [batch, doc_count] or null
    const float* lexical_max = nullptr;  // [batch]
    float dense_weight = 1.0f;
};

// Rows per work item and workgroup count used by the VALU scan for this corpus/batch.
struct ValuShape {
    int lanes = 1;
    int block_rows = 64;
    int workgroups = 1;
    int query_group = 1;  // queries staged per launch
};
ValuShape valuShape(const ScanArgs& scan);
int launchValuScan(const ScanArgs& scan, const PhaseArgs& phase, const EmitArgs& emit,
                   int workgroups, hipStream_t stream);

// The int8 x int8 MFMA scan (per-vector mode, dim in {256, 384, 512, 768, 1024}).
bool mfmaSupported(const ScanArgs& scan);
constexpr int kMfmaBlockRows = 64;
int mfmaWorkgroups();
// Candidate segments per workgroup of the int8 MFMA scan (one per row half of a query's lanes).
int mfmaSegmentsPerWorkgroup();
int launchMfmaScan(const ScanArgs& scan, const PhaseArgs& phase, const EmitArgs& emit,
                   int workgroups, hipStream_t stream);

// The float32 / float16 MFMA scan (batches of at least 4 queries, cosine or dot, no mask, dim in
// {128, 256, 384, 512}; lexical scores are fused); block rows depend on the row size.
bool mfmaFloatSupported(const ScanArgs& scan);
int mfmaFloatBlockRows(const ScanArgs& scan);
int launchMfmaFloatScan(const ScanArgs& scan, const PhaseArgs& phase, const EmitArgs& emit,
                        int workgroups, hipStream_t stream);

// The float32 scan on the bf16 matrix cores (fused_mfma_split.hip): three-part bf16 splits of
// rows and queries, for launches of 32 to 128 queries over rows of 256 or 384 dims (32-row
// tiles, as the float MFMA scan uses at those sizes); launchMfmaFloatScan hands it those launches.
bool mfmaSplitSupported(const ScanArgs& scan, int queries_in_launch);
int launchMfmaSplitScan(const ScanArgs& scan, const PhaseArgs& phase, const EmitArgs& emit, int workgroups,
                        int q0, int count, hipStream_t stream);

// The binary (Hamming) MFMA scan (batches of at least 4 queries, no mask or lexical scores,
// dim 512 or 1024).
bool mfmaBinarySupported(const ScanArgs& scan);
int mfmaBinaryBlockRows(const ScanArgs& scan);
// Whether the binary scan can take the sketch plan (its streaming kernel has the sketch and rerun
// modes, one launch per set of 32 queries, at any batch size); its sketch slots per workgroup.
bool mfmaBinaryStreams(const ScanArgs& scan);
int mfmaBinarySketchSlotsPerWorkgroup();
int launchMfmaBinaryScan(const ScanArgs& scan, const PhaseArgs& phase, const EmitArgs& emit,
                         int workgroups, hipStream_t stream);

// Single-pass scan (single_pass.hip) for at most kSinglePassQueries queries and a selection of at
// most kMaxK keys: each of `workgroups` workgroups writes its exact top-`width` of every query to
// a candidate segment. Workgroup b is segment s = b / groups of merge query q * groups + b %
// groups, i.e. seg[((s * batch * groups + q * groups + b % groups) << seg_log2) + j], j <
// seg_count[s * batch * groups + q * groups + b % groups], so one selectMerge over the batch *
// groups merge queries (workgroups / groups segments each) takes every group's top-width, and
// with groups > 1 merges of up to 8 neighbouring group results at a time finish. Nothing
// overflows.
constexpr int kSinglePassQueries = 4;
constexpr long long kSinglePassMergeKeys = 12288;  // candidate keys the merge gathers in LDS (topk.hip)
struct SinglePassArgs {
    int width = 0;
    int workgroups = 0;
    int cap = 0;     // LDS list keys per query (singlePassShape)
    int groups = 1;  // merge groups (singlePassShape)
    std::uint64_t* seg = nullptr;
    std::uint32_t* seg_count = nullptr;
    int seg_log2 = 0;
};
struct SinglePassShape {
    bool supported = false;
    int workgroups = 0;
    int cap = 0;
    int groups = 1;
    int seg_log2 = 0;
};
SinglePassShape singlePassShape(const ScanArgs& scan, int width);
bool singlePassSupported(const ScanArgs& scan, int width);
int launchSinglePass(const ScanArgs& scan, const SinglePassArgs& args, hipStream_t stream);

// Exact device fallback (recover.hip): the top-`width` of every query whose flag is set (every
// query with `force`; the listed queries in list mode) over the whole corpus, written sorted to
// out_keys [batch, width] and, when out_index is set, as (index, score) pairs [batch, width].
// The scan arguments are the VALU scan's: original row scales and allow-mask, device-prepared
// queries, lexical scores.
struct RecoverArgs {
    const std::uint32_t* flags = nullptr;
    bool force = false;
    int width = 0;
    std::uint64_t* out_keys = nullptr;
    int* out_index = nullptr;
    float* out_score = nullptr;
    // List mode (flag_list set, force clear): block e takes the e-th flagged query
    // flag_list[e], e < *flag_count. With `seg` set, the rerun (EmitArgs::q_list) wrote entry
    // e's keys to its segments (n_seg of them, rerunSegLog2(seg_log2, batch, F) slots each);
    // when none overflowed, the query's selection is taken from them and the corpus is not
    // read again.
    const std::uint32_t* flag_list = nullptr;
    const std::uint32_t* flag_count = nullptr;
    const std::uint64_t* seg = nullptr;
    const std::uint32_t* seg_count = nullptr;
    int n_seg = 0;
    int seg_log2 = 0;
};
bool recoverSupported(const ScanArgs& scan);
int launchRecover(const ScanArgs& scan, const RecoverArgs& args, hipStream_t stream);
// The final merge of a phased search fused with its exact fallback (not the list mode): one launch
// of `batch` blocks, each merging its query as launchSelectMerge does (no threshold output) and,
// when the merge flags the query or args.force is set, recomputing its selection as the last
// resort of launchRecover does. args.width must equal k.
int launchMergeRecover(const MergeInputs& in, int k, int batch, std::uint64_t* out_keys, std::uint32_t* overflow,
                       int* out_index, float* out_score, const ScanArgs& scan, const RecoverArgs& args,
                       hipStream_t stream);

}  // namespace zcgvs_hip
