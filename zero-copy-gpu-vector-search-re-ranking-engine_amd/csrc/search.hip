// Fused search pipeline (zcgvs_search_topk): the device stages of src/search/searcher.cpp:209-285
// without the [batch, N] score matrix.
//
//   1. query preparation: sign packing for a binary corpus (searcher.cpp:215-218), per-row int8
//      quantization for the per-vector int8 mode;
//   2. optional BM25 scores and their per-query maximum (hybrid, searcher.cpp:235-259);
//   3. the scan selects `width` = rescore_candidates (rescore on) or k keys per query, either
//      - in one pass (single_pass.hip: at most 4 queries, no MFMA scan applies): per-workgroup
//        exact top-width lists, then one merge (two for wide selections); or
//      - in phases (fused.hpp): a dense sample, then threshold phases that emit only keys above
//        the running threshold, with a per-query merge after every phase, followed by the exact
//        fallback (recover.hip) for any query whose candidate segments overflowed, so the result
//        is exact for every input;
//   4. optional exact gather rescore of those candidates and a final top-k, whose keys carry the
//      corpus id, which subsumes the reference's remap (searcher.cpp:261-278).
//
// Shapes the fused kernels do not take (rows that are not whole 16-byte chunks, very wide rows)
// run the materialized launchers instead: zcgvs_launch_similarity into a workspace score matrix,
// then zcgvs_launch_topk, exactly the reference's stage order.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <string>
#include <vector>

#include "common.hpp"
#include "fused.hpp"
#include "rescore.hpp"
#include "select.hpp"

namespace zcgvs_hip {

bool valuSupported(const ScanArgs& scan);

namespace {

constexpr std::size_t kAlign = 256;
// Each threshold phase visits up to `growth` times as many rows as all phases before it, so it
// yields about width * growth candidates per query on a corpus in random order. The growth is 8,
// or larger while batch * width * growth stays within kCandidateBudget keys and one query's
// candidates fit the merge's LDS gather (small batches and k then need only a dense sample and
// one threshold phase).
constexpr long long kPhaseGrowth = 8;
constexpr long long kCandidateBudget = 1LL << 18;
constexpr long long kMergeLdsKeys = 12288;  // candidate keys a query's merge gathers in LDS (topk.hip)

std::size_t alignUp(std::size_t value) { return (value + kAlign - 1) / kAlign * kAlign; }

int ceilLog2(long long value) {
    int bits = 0;
    while ((1LL << bits) < value) {
        ++bits;
    }
    return bits;
}

struct Layout {
    std::size_t total = 0;
    std::size_t add(std::size_t bytes) {
        const std::size_t offset = total;
        total += alignUp(std::max<std::size_t>(bytes, 1));
        return offset;
    }
};

struct Plan {
    int status = ZCGVS_OK;
    std::string error;

    bool binary = false;
    bool per_vector = false;
    bool hybrid = false;
    bool rescore = false;
    bool materialized = false;
    bool use_mfma = false;
    bool use_mfma_float = false;
    bool use_mfma_binary = false;
    bool direct_scales = false;  // MFMA path without a mask: only the tail tile's scales are copied
    bool lex_sorted = false;     // hybrid with postings ascending by document: sliced BM25 stage
    bool recover = false;        // threshold phases ran: the exact fallback follows them
    // int8 MFMA scan or binary streaming scan over a large corpus: a sketch phase and one
    // speculative full scan instead of the threshold phases (see makePlan)
    bool sketch = false;
    int sketch_slots = 0;        // sketch slots (2 per workgroup int8, 8 binary)
    int sketch_rank = 0;         // tau = the sketch_rank-th best slot score
    // the scan kernel reruns the flagged queries over the whole corpus before the fallback
    bool rerun = false;
    int rerun_seg_log2 = 0;      // the segments' normal capacity (the test flag shrinks seg_log2 only)
    PhaseArgs full;              // every block of the corpus (the rerun's phase)
    bool single_pass = false;    // a few queries: one scan launch and one or two merges
    int sp_cap = 0;              // single pass: LDS list keys per query
    int sp_groups = 1;           // single pass: merge groups (a second merge when above 1)
    int width = 0;  // keys selected by the scan stage
    int block_rows = 64;
    int workgroups = 1;
    int segments = 1;  // candidate segments per query of a threshold phase
    int seg_log2 = 5;
    long long dense_stride = 0;
    std::vector<PhaseArgs> phases;

    // workspace offsets
    std::size_t mscales = 0;  // MFMA path: row scales padded to whole tiles, NaN = masked/padding
    std::size_t qbits = 0, qi8 = 0, qscale = 0, lex = 0, lexmax = 0, dense = 0, seg = 0,
                segcnt = 0, keys = 0, tau = 0, overflow = 0, rescored = 0, scores = 0, lexmat = 0,
                topk_a = 0, topk_b = 0, topk_c = 0, topk_d = 0, cand_idx = 0, cand_val = 0, sp_level = 0,
                local_idx = 0, rescore_val = 0, lexmax_m = 0, lexbounds = 0, sketchbuf = 0, tau_safe = 0,
                flag_list = 0, flag_count = 0;
    std::size_t total = 0;
};

Plan fail(int status, const std::string& message) {
    Plan plan;
    plan.status = status;
    plan.error = message;
    return plan;
}

// Argument checks of src/search/searcher.cpp:91-135, plus the descriptor's own consistency.
Plan validate(const zcgvs_search_desc& d) {
    const zcgvs_store_desc& c = d.corpus;
    if (c.data == nullptr || d.queries == nullptr) {
        return fail(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: corpus and queries must be device pointers");
    }
    if (c.dim <= 0) {
        return fail(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: corpus dim must be positive");
    }
    if (!validDtype(c.dtype)) {
        return fail(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: unknown corpus dtype");
    }
    if (!validMetric(d.metric)) {
        return fail(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: unknown metric");
    }
    if (d.batch <= 0) {
        return fail(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: batch must be positive");
    }
    if (d.k <= 0) {
        return fail(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: k must be positive");
    }
    if (c.doc_count > static_cast<std::int64_t>(INT32_MAX)) {
        return fail(ZCGVS_ERR_RUNTIME, "zcgvs: corpus exceeds the supported document count");
    }
    if (c.doc_count <= 0) {
        return fail(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: corpus is empty");
    }
    if (d.k > c.doc_count) {
        return fail(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: k=" + std::to_string(d.k) +
                                                    " exceeds corpus size " +
                                                    std::to_string(c.doc_count));
    }
    if (d.k > kMaxK) {
        return fail(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: k=" + std::to_string(d.k) +
                                                    " exceeds kernel capacity " +
                                                    std::to_string(kMaxK));
    }
    Plan plan;
    plan.binary = c.dtype == ZCGVS_DTYPE_BINARY;
    plan.per_vector = c.dtype == ZCGVS_DTYPE_I8 && d.int8_mode == ZCGVS_INT8_PER_VECTOR;
    if (c.dtype == ZCGVS_DTYPE_I8 && d.int8_mode != ZCGVS_INT8_REFERENCE &&
        d.int8_mode != ZCGVS_INT8_PER_VECTOR) {
        return fail(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: unknown int8 mode");
    }
    if (plan.per_vector) {
        if (c.row_scales == nullptr) {
            return fail(ZCGVS_ERR_INVALID_ARGUMENT,
                        "zcgvs: per-vector int8 mode needs the corpus row scales");
        }
        if (d.metric == ZCGVS_METRIC_L2) {
            return fail(ZCGVS_ERR_INVALID_ARGUMENT,
                        "zcgvs: per-vector int8 mode supports cosine and dot only");
        }
    }
    plan.rescore = d.rescore.data != nullptr && d.rescore_candidates > 0;
    if (plan.rescore) {
        if (d.rescore_candidates < d.k) {
            return fail(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: rescore_candidates must be at least k");
        }
        if (d.rescore_candidates > c.doc_count) {
            return fail(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: rescore_candidates exceeds corpus size");
        }
        if (d.rescore_candidates > kMaxK) {
            return fail(ZCGVS_ERR_INVALID_ARGUMENT,
                        "zcgvs: rescore_candidates=" + std::to_string(d.rescore_candidates) +
                            " exceeds kernel capacity " + std::to_string(kMaxK));
        }
        if (d.rescore.dtype == ZCGVS_DTYPE_BINARY || !validDtype(d.rescore.dtype)) {
            return fail(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: rescore store must not be binary");
        }
        if (d.rescore.dim != c.dim) {
            return fail(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: rescore store dim does not match the corpus");
        }
        if (d.rescore.doc_count < c.doc_count) {
            return fail(ZCGVS_ERR_INVALID_ARGUMENT,
                        "zcgvs: rescore store holds fewer documents than the corpus");
        }
    }
    plan.hybrid = d.query_terms != nullptr && d.lexical_stride > 0;
    if ((d.flags & ZCGVS_SEARCH_SORTED_POSTINGS) != 0 && (d.flags & ZCGVS_SEARCH_UNSORTED_POSTINGS) != 0) {
        return fail(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: postings cannot be both sorted and unsorted");
    }
    if (plan.hybrid) {
        if (d.lex_offsets == nullptr || d.lex_docs == nullptr || d.lex_weights == nullptr) {
            return fail(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: lexical index pointers are null");
        }
        if (d.lex_vocab_size <= 0) {
            return fail(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: lexical vocabulary size must be positive");
        }
        if (d.lex_doc_count < c.doc_count) {
            return fail(ZCGVS_ERR_INVALID_ARGUMENT,
                        "zcgvs: lexical index holds fewer documents than the corpus");
        }
        if (d.lex_slice_table != nullptr && (d.flags & ZCGVS_SEARCH_SORTED_POSTINGS) == 0) {
            return fail(ZCGVS_ERR_INVALID_ARGUMENT,
                        "zcgvs: a lexical slice table needs ZCGVS_SEARCH_SORTED_POSTINGS");
        }
        if (d.lex_slice_table != nullptr && d.lex_doc_count > INT32_MAX) {
            return fail(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: a lexical slice table covers at most 2^31 - 1 documents");
        }
    }
    return plan;
}

ScanArgs scanArgsOf(const zcgvs_search_desc& d, const Plan& plan, std::uint8_t* ws) {
    ScanArgs scan;
    scan.corpus = d.corpus.data;
    scan.doc_count = d.corpus.doc_count;
    scan.dim = d.corpus.dim;
    scan.dtype = d.corpus.dtype;
    scan.scale = d.corpus.scale;
    scan.batch = d.batch;
    scan.metric = d.metric;
    scan.mask = d.mask;
    scan.queries = d.queries;
    if (plan.per_vector) {
        scan.row_scales = d.corpus.row_scales;
        if (plan.use_mfma) {
            const float* staged = ws != nullptr ? reinterpret_cast<const float*>(ws + plan.mscales) : nullptr;
            if (plan.direct_scales) {
                scan.tail_scales = staged;
            } else {
                scan.row_scales = staged;
            }
            scan.mask = nullptr;
        }
        scan.queries = ws != nullptr ? ws + plan.qi8 : nullptr;
        scan.query_scales = ws != nullptr ? reinterpret_cast<const float*>(ws + plan.qscale) : nullptr;
    }
    if (plan.binary) {
        scan.queries = ws != nullptr ? ws + plan.qbits : nullptr;
    }
    if (plan.hybrid) {
        scan.lexical = ws != nullptr ? reinterpret_cast<const float*>(ws + plan.lex) : nullptr;
        scan.lexical_max = ws != nullptr ? reinterpret_cast<const float*>(ws + plan.lexmax) : nullptr;
        scan.dense_weight = d.dense_weight;
    }
    return scan;
}

// The scan arguments of the exact fallback: those of the VALU scan (the caller's row scales and
// allow-mask, never the MFMA scan's padded scale copy).
ScanArgs recoverArgsOf(const zcgvs_search_desc& d, const Plan& plan, std::uint8_t* ws) {
    Plan valu = plan;
    valu.use_mfma = false;
    ScanArgs scan = scanArgsOf(d, valu, ws);
    scan.row_scales = plan.per_vector ? d.corpus.row_scales : nullptr;
    scan.tail_scales = nullptr;
    scan.mask = d.mask;
    return scan;
}

Plan makePlan(const zcgvs_search_desc& d) {
    Plan plan = validate(d);
    if (plan.status != ZCGVS_OK) {
        return plan;
    }
    const long long n = d.corpus.doc_count;
    const int batch = d.batch;
    const int dim = d.corpus.dim;
    plan.width = plan.rescore ? d.rescore_candidates : d.k;

    // Probe the scan engine with a dummy aligned pointer set (alignment is re-checked at run).
    ScanArgs probe = scanArgsOf(d, plan, nullptr);
    if (plan.per_vector || plan.binary) {
        probe.queries = reinterpret_cast<const void*>(static_cast<std::uintptr_t>(kAlign));
    }
    if (plan.per_vector) {
        probe.query_scales = reinterpret_cast<const float*>(static_cast<std::uintptr_t>(kAlign));
        probe.mask = nullptr;  // an allow-mask is merged into the row scales for the MFMA scan
    }
    if (plan.hybrid) {
        probe.lexical = reinterpret_cast<const float*>(static_cast<std::uintptr_t>(kAlign));
    }
    const bool forced = (d.flags & ZCGVS_SEARCH_MATERIALIZE) != 0;
    plan.use_mfma = !forced && mfmaSupported(probe);
    plan.use_mfma_float = !forced && !plan.use_mfma && mfmaFloatSupported(probe);
    plan.use_mfma_binary = !forced && mfmaBinarySupported(probe);
    plan.materialized = forced || (!plan.use_mfma && !plan.use_mfma_float && !plan.use_mfma_binary &&
                                   !valuSupported(probe));
    if (!plan.materialized) {
        ScanArgs fallback = probe;
        fallback.row_scales = plan.per_vector ? d.corpus.row_scales : nullptr;
        fallback.mask = d.mask;
        if (!recoverSupported(fallback)) {
            plan.materialized = true;  // no exact fallback for this row layout
            plan.use_mfma = plan.use_mfma_float = plan.use_mfma_binary = false;
        }
    }
    if (plan.per_vector && plan.materialized && dim % 16 != 0) {
        return fail(ZCGVS_ERR_INVALID_ARGUMENT,
                    "zcgvs: per-vector int8 mode needs dim % 16 == 0 and a 16-byte aligned corpus");
    }

    Layout layout;
    if (plan.binary) {
        plan.qbits = layout.add(static_cast<std::size_t>(batch) * binaryWords(dim) * 4);
    }
    if (plan.per_vector) {
        plan.qi8 = layout.add(static_cast<std::size_t>(batch) * dim);
        plan.qscale = layout.add(static_cast<std::size_t>(batch) * 4);
        if (plan.use_mfma) {
            // Without a mask the scan reads the caller's scales and needs a padded copy of the
            // last tile's only; with one, masked rows get NaN in a padded copy of all scales.
            plan.direct_scales = d.mask == nullptr && aligned16(d.corpus.row_scales);
            const long long tiles = (n + kMfmaBlockRows - 1) / kMfmaBlockRows;
            plan.mscales = layout.add(static_cast<std::size_t>(plan.direct_scales ? 1 : tiles) * kMfmaBlockRows * 4);
        }
    }
    plan.overflow = layout.add(static_cast<std::size_t>(batch) * 4);
    if (plan.hybrid && (d.flags & ZCGVS_SEARCH_SORTED_POSTINGS) != 0) {
        plan.lex_sorted = true;
        plan.lexbounds = layout.add(lexicalBoundsBytes(batch, d.lexical_stride, static_cast<int>(n)));
    }

    if (plan.materialized) {
        // Reference-order pipeline over a workspace score matrix.
        const std::size_t elements = static_cast<std::size_t>(batch) * n;
        plan.scores = layout.add(elements * 4);
        if (plan.hybrid) {
            plan.lexmat = layout.add(elements * 4);
            plan.lexmax_m = layout.add(static_cast<std::size_t>(batch) * 4);
        }
        const std::size_t scratch = static_cast<std::size_t>(batch) *
                                    zcgvs_topk_scratch_elements(static_cast<int>(n), plan.width) * 4;
        plan.topk_a = layout.add(scratch);
        plan.topk_b = layout.add(scratch);
        plan.topk_c = layout.add(scratch);
        plan.topk_d = layout.add(scratch);
        if (plan.rescore) {
            const std::size_t cands = static_cast<std::size_t>(batch) * plan.width;
            plan.cand_idx = layout.add(cands * 4);
            plan.cand_val = layout.add(cands * 4);
            plan.rescore_val = layout.add(cands * 4);
            plan.local_idx = layout.add(static_cast<std::size_t>(batch) * d.k * 4);
            // C candidates per query need their own top-k scratch.
            const std::size_t s2 = static_cast<std::size_t>(batch) *
                                   zcgvs_topk_scratch_elements(plan.width, d.k) * 4;
            if (s2 > scratch) {
                return fail(ZCGVS_ERR_RUNTIME, "zcgvs: rescore scratch sizing");
            }
        }
        plan.total = layout.total;
        return plan;
    }

    // A few queries and no MFMA scan: one launch streams the corpus once and keeps each
    // workgroup's exact top-width (single_pass.hip), so neither threshold phases nor the fallback
    // run. (Not with the test flags, which exercise the phased scan's fallback.)
    SinglePassShape single_shape;
    if (!plan.use_mfma && !plan.use_mfma_float && !plan.use_mfma_binary &&
        (d.flags & (ZCGVS_SEARCH_FORCE_EXACT_PASS | ZCGVS_SEARCH_TEST_TINY_SEGMENTS)) == 0) {
        ScanArgs single = probe;
        single.row_scales = plan.per_vector ? d.corpus.row_scales : nullptr;
        single.mask = d.mask;
        single_shape = singlePassShape(single, plan.width);
        plan.single_pass = single_shape.supported;
    }
    if (plan.single_pass) {
        plan.workgroups = single_shape.workgroups;
        plan.segments = plan.workgroups;
        plan.block_rows = 1;
        plan.seg_log2 = single_shape.seg_log2;
        plan.sp_cap = single_shape.cap;
        plan.sp_groups = single_shape.groups;
        PhaseArgs whole;
        whole.items = n;
        whole.block_rows = 1;
        whole.dense = 0;
        plan.phases.push_back(whole);
        if (plan.hybrid) {
            plan.lex = layout.add(static_cast<std::size_t>(batch) * n * 4);
            plan.lexmax = layout.add(static_cast<std::size_t>(batch) * 4);
        }
        plan.seg = layout.add((static_cast<std::size_t>(plan.segments) * batch << plan.seg_log2) * 8);
        plan.segcnt = layout.add(static_cast<std::size_t>(plan.segments) * batch * 4);
        if (plan.sp_groups > 1) {
            // two buffers of every (query, group) result, merged 8 groups at a time in turn
            plan.sp_level = layout.add(2 * static_cast<std::size_t>(batch) * plan.sp_groups * plan.width * 8);
        }
        plan.keys = layout.add(static_cast<std::size_t>(batch) * plan.width * 8);
        if (plan.rescore) {
            plan.rescored = layout.add(static_cast<std::size_t>(batch) * plan.width * 8);
        }
        plan.total = layout.total;
        return plan;
    }

    if (plan.use_mfma) {
        plan.block_rows = kMfmaBlockRows;
        plan.workgroups = mfmaWorkgroups();
    } else if (plan.use_mfma_float) {
        plan.block_rows = mfmaFloatBlockRows(probe);
        plan.workgroups = mfmaWorkgroups();
    } else if (plan.use_mfma_binary) {
        plan.block_rows = mfmaBinaryBlockRows(probe);
        plan.workgroups = mfmaWorkgroups();
    } else {
        const ValuShape shape = valuShape(probe);
        plan.block_rows = shape.block_rows;
        plan.workgroups = shape.workgroups;
    }

    // Phase schedule: phase 0 samples ~max(8 * width, 4096) rows densely (for wide selections
    // that keeps its keys within the merge's LDS capacity); each later phase
    // visits up to growth_cap times as many blocks as all phases before it.
    long long growth_cap = kPhaseGrowth;
    // A phase yields about width * growth candidates per query; beyond kMergeLdsKeys (with the
    // width keys kept from before) a query's merge walks its segments in global memory, once per
    // radix pass, which costs far more than one more phase.
    while (growth_cap * 2 * batch * plan.width <= kCandidateBudget &&
           (growth_cap * 2 + 1) * plan.width <= kMergeLdsKeys) {
        growth_cap *= 2;
    }
    const long long blocks = (n + plan.block_rows - 1) / plan.block_rows;
    const long long target_rows = std::max<long long>(8LL * plan.width, 4096);
    const long long blocks0 = (target_rows + plan.block_rows - 1) / plan.block_rows;
    long long stride = 1;
    while ((blocks + 2 * stride - 1) / (2 * stride) >= blocks0) {
        stride *= 2;
    }
    PhaseArgs first;
    first.stride = stride;
    first.skip = 0;
    first.items = phaseItems(blocks, stride, 0);
    first.dense = 1;
    first.block_rows = plan.block_rows;
    plan.phases.push_back(first);
    long long growth = 1;
    while (stride > 1) {
        const long long next = std::max<long long>(1, stride / growth_cap);
        PhaseArgs phase;
        phase.stride = next;
        phase.skip = stride / next;
        phase.items = phaseItems(blocks, next, phase.skip);
        phase.dense = 0;
        phase.block_rows = plan.block_rows;
        growth = std::max(growth, phase.skip);
        plan.phases.push_back(phase);
        stride = next;
    }
    plan.dense_stride = first.items * plan.block_rows;
    plan.segments = plan.workgroups * (plan.use_mfma ? mfmaSegmentsPerWorkgroup() : 1);
    plan.full.stride = 1;
    plan.full.skip = 0;
    plan.full.items = blocks;
    plan.full.block_rows = plan.block_rows;
    // (the binary scan runs the sketch and the rerun in its streaming kernel, one launch per set of 32
    // queries; its full scan streams too for one set and runs the tile kernel beyond)
    const bool binary_sketch = plan.use_mfma_binary && mfmaBinaryStreams(probe);
    plan.rerun = plan.use_mfma;
    // Segment capacity: 4x the expected candidates per (segment, query) of the widest phase.
    long long expected = (static_cast<long long>(plan.width) * growth) / plan.segments;

    // Sketch plan (int8 MFMA scan and binary streaming scan, when the threshold phases would be
    // three or more): a sketch phase over every 32nd block (64th for the binary scan) keeps per
    // slot (a row half of a workgroup's lanes in the int8 scan, a pair of wavefronts in the binary
    // one) the best exact score of each query; the j-th best of those slot scores is the threshold
    // of ONE scan over the whole corpus. With f = sketch rows / corpus rows, the number of
    // corpus rows at or above the sketch's j-th best score is about Gamma(j) / f, so
    // j = width f + 5.5 sqrt(width f) + 2 (15 at f = 1/32, width = 100) leaves fewer than width
    // such rows with probability about 1e-6 per query (Poisson tail), while the scan emits about
    // j / f candidates per query. The merge flags a query for the fallback when fewer than width
    // candidates reached it; the k-th best slot score is its guaranteed threshold then.
    const int slots = (plan.use_mfma ? 2 : mfmaBinarySketchSlotsPerWorkgroup()) * plan.workgroups;
    // (A smaller corpus samples every 16th, 8th or 4th block, so every workgroup still sees at
    // least 4 sampled blocks; below that the threshold phases stay. The binary scan samples half
    // as many blocks at full size: its sketch launch costs more per row than its full scan, and at
    // binary 50M x 1024, B = 32, width 1000 the 64th-block sketch took the step from 1.49-1.50 to
    // 1.47-1.48 ms; the int8 scan timed the same at 32 and 64.)
    long long sketch_stride = binary_sketch ? 64 : 32;
    while (sketch_stride > 4 && phaseItems(blocks, sketch_stride, 0) < 4LL * plan.workgroups) {
        sketch_stride /= 2;
    }
    if ((plan.use_mfma || binary_sketch) && plan.phases.size() >= 3 && slots <= kMaxSketchSlots &&
        slots >= plan.width &&
        phaseItems(blocks, sketch_stride, 0) >= 4LL * plan.workgroups) {
        PhaseArgs sketch;
        sketch.stride = sketch_stride;
        sketch.skip = 0;
        sketch.items = phaseItems(blocks, sketch_stride, 0);
        sketch.sketch = 1;
        sketch.block_rows = plan.block_rows;
        const double f = static_cast<double>(sketch.items) / static_cast<double>(blocks);
        const double kf = plan.width * f;
        const int j = static_cast<int>(std::ceil(kf + 5.5 * std::sqrt(kf) + 2.0));
        plan.sketch = true;
        plan.rerun = true;
        plan.sketch_slots = slots;
        plan.sketch_rank = std::max(1, std::min({j, plan.width, slots}));
        if ((d.flags & ZCGVS_SEARCH_TEST_HIGH_THRESHOLD) != 0) {
            plan.sketch_rank = 1;  // tests: most queries find fewer than width keys above it
        }
        plan.phases.clear();
        plan.phases.push_back(sketch);
        plan.phases.push_back(plan.full);
        plan.dense_stride = 0;
        expected = static_cast<long long>(std::ceil(plan.sketch_rank / f)) / plan.segments;
    }
    // At least one full work item of candidates (two tiles of the int8 MFMA scan, whose segments
    // take half a tile's rows each) per segment, so a corpus whose best rows sit together in a few
    // blocks (sorted or clustered rows) does not overflow the segments.
    const long long item_rows = plan.use_mfma ? kMfmaBlockRows : plan.block_rows;
    // (at most 2^23 slots: the int8 MFMA scan packs a slot, a half and an 8-bit query into 32 bits)
    plan.seg_log2 = std::min(23, std::max({6, ceilLog2(4 * expected + 16), ceilLog2(item_rows)}));
    plan.rerun_seg_log2 = plan.seg_log2;
    if ((d.flags & ZCGVS_SEARCH_TEST_TINY_RERUN) != 0) {
        plan.rerun_seg_log2 = 1;  // tests: the reruns overflow as well (see the flag)
    }
    if ((d.flags & ZCGVS_SEARCH_TEST_TINY_SEGMENTS) != 0) {
        plan.seg_log2 = 1;  // tests: overflow nearly every query so the fallback runs from its flags
    }
    plan.recover = plan.phases.size() > 1 || (d.flags & ZCGVS_SEARCH_FORCE_EXACT_PASS) != 0;

    if (plan.hybrid) {
        plan.lex = layout.add(static_cast<std::size_t>(batch) * n * 4);
        plan.lexmax = layout.add(static_cast<std::size_t>(batch) * 4);
    }
    plan.dense = layout.add(static_cast<std::size_t>(batch) * plan.dense_stride * 8);
    if (plan.phases.size() > 1) {
        // (the rerun shares the buffer at the normal capacity, which the test flag may lower
        // for the first attempt)
        const int seg_bits = plan.rerun ? std::max(plan.seg_log2, plan.rerun_seg_log2) : plan.seg_log2;
        plan.seg = layout.add((static_cast<std::size_t>(plan.segments) * batch << seg_bits) * 8);
        plan.segcnt = layout.add(static_cast<std::size_t>(plan.segments) * batch * 4);
    }
    plan.keys = layout.add(static_cast<std::size_t>(batch) * plan.width * 8);
    plan.tau = layout.add(static_cast<std::size_t>(batch) * 8);
    plan.flag_list = layout.add(static_cast<std::size_t>(batch) * 4);
    plan.flag_count = layout.add(4);
    if (plan.sketch) {
        plan.sketchbuf = layout.add(static_cast<std::size_t>(plan.sketch_slots) * batch * 4);
        plan.tau_safe = layout.add(static_cast<std::size_t>(batch) * 8);
    }
    if (plan.rescore) {
        plan.rescored = layout.add(static_cast<std::size_t>(batch) * plan.width * 8);
    }
    plan.total = layout.total;
    return plan;
}

template <typename T>
T* at(std::uint8_t* ws, std::size_t offset) {
    return reinterpret_cast<T*>(ws + offset);
}

int runMaterialized(const zcgvs_search_desc& d, const Plan& plan, std::uint8_t* ws, int* out_idx,
                    float* out_val, hipStream_t stream) {
    const int n = static_cast<int>(d.corpus.doc_count);
    const int batch = d.batch;
    float* scores = at<float>(ws, plan.scores);
    int status = ZCGVS_OK;
    zcgvs_stream_t s = stream;
    if (plan.per_vector) {
        status = zcgvs_launch_similarity_i8i8(static_cast<const std::int8_t*>(d.corpus.data),
                                              d.corpus.row_scales, n, d.corpus.dim,
                                              at<std::int8_t>(ws, plan.qi8),
                                              at<float>(ws, plan.qscale), batch, d.mask, d.metric,
                                              scores, s);
    } else {
        const void* queries = plan.binary ? static_cast<const void*>(ws + plan.qbits)
                                          : static_cast<const void*>(d.queries);
        status = zcgvs_launch_similarity(d.corpus.data, d.corpus.dtype, d.corpus.scale, n,
                                         d.corpus.dim, queries, batch, d.mask, d.metric, scores, s);
    }
    if (status != ZCGVS_OK) {
        return status;
    }
    if (plan.hybrid) {
        float* lexical = at<float>(ws, plan.lexmat);
        float* lexmax = at<float>(ws, plan.lexmax_m);
        status = launchLexicalScores(d.lex_offsets, d.lex_docs, d.lex_weights, d.lex_vocab_size, d.query_terms,
                                     d.lexical_stride, batch, n, lexical, lexmax,
                                     plan.lex_sorted ? at<std::int64_t>(ws, plan.lexbounds) : nullptr,
                                     d.lex_slice_table, d.lex_doc_count, stream);
        if (status != ZCGVS_OK) {
            return status;
        }
        for (int q = 0; q < batch; ++q) {
            status = zcgvs_launch_fuse_scores(scores + static_cast<std::size_t>(q) * n,
                                              lexical + static_cast<std::size_t>(q) * n,
                                              lexmax + q, d.dense_weight, n, s);
            if (status != ZCGVS_OK) {
                return status;
            }
        }
    }
    float* sa = at<float>(ws, plan.topk_a);
    int* ia = at<int>(ws, plan.topk_b);
    float* sb = at<float>(ws, plan.topk_c);
    int* ib = at<int>(ws, plan.topk_d);
    if (!plan.rescore) {
        return zcgvs_launch_topk(scores, n, d.k, batch, out_idx, out_val, sa, ia, sb, ib, s);
    }
    const int c = plan.width;
    int* cand_idx = at<int>(ws, plan.cand_idx);
    float* cand_val = at<float>(ws, plan.cand_val);
    float* rescored = at<float>(ws, plan.rescore_val);
    int* local = at<int>(ws, plan.local_idx);
    status = zcgvs_launch_topk(scores, n, c, batch, cand_idx, cand_val, sa, ia, sb, ib, s);
    if (status != ZCGVS_OK) {
        return status;
    }
    status = zcgvs_launch_gather_rescore(d.rescore.data, d.rescore.dtype, d.rescore.scale,
                                         static_cast<int>(d.rescore.doc_count), d.corpus.dim,
                                         d.queries, batch, cand_idx, c, d.metric, rescored, s);
    if (status != ZCGVS_OK) {
        return status;
    }
    status = zcgvs_launch_topk(rescored, c, d.k, batch, local, out_val, sa, ia, sb, ib, s);
    if (status != ZCGVS_OK) {
        return status;
    }
    return zcgvs_launch_remap_indices(cand_idx, local, c, d.k, batch, out_idx, s);
}

// The MFMA scan's row scales: the corpus scales padded to `padded` rows, with NaN (its
// masked-row marker) for rows the allow-mask excludes and for the padding.
// out[i] = scales[first + i] for allowed rows below n, NaN otherwise, for i < count.
__global__ void mergeMaskedScalesKernel(const float* __restrict__ scales,
                                        const std::uint8_t* __restrict__ mask, long long n,
                                        long long first, long long count, float* __restrict__ out) {
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += stride) {
        const long long row = first + i;
        const bool allowed = row < n && (mask == nullptr || mask[row] != 0);
        out[i] = allowed ? scales[row] : __uint_as_float(0x7FC00000u);
    }
}

__global__ void zeroWordsKernel(std::uint32_t* __restrict__ dst, std::size_t count) {
    const std::size_t stride = static_cast<std::size_t>(gridDim.x) * blockDim.x;
    for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
         i < count; i += stride) {
        dst[i] = 0u;
    }
}

// Workspace of zcgvs_search_topk_noalloc: one library-owned array per device, so a caller that
// cannot allocate still runs the pipeline. Its size caps the searches that entry point accepts.
constexpr std::size_t kStaticScratchBytes = std::size_t(64) << 20;

}  // namespace

}  // namespace zcgvs_hip

// In host code `scratch` names a host-side stand-in, not device memory: its device address comes
// from hipGetSymbolAddress, once per device (scratchAddress below).
static __device__ __align__(256) std::uint8_t scratch[zcgvs_hip::kStaticScratchBytes];

namespace zcgvs_hip {

namespace {

std::mutex g_scratch_mutex;
std::vector<void*> g_scratch_address;  // indexed by device; null until first looked up

// Device address of this device's `scratch`, looked up with that device current on its first use.
int scratchAddress(void** address) {
    int device = 0;
    ZCGVS_HIP_RETURN(hipGetDevice(&device));
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (static_cast<int>(g_scratch_address.size()) <= device) {
        g_scratch_address.resize(static_cast<std::size_t>(device) + 1, nullptr);
    }
    void*& cached = g_scratch_address[static_cast<std::size_t>(device)];
    if (cached == nullptr) {
        void* found = nullptr;
        const hipError_t status = hipGetSymbolAddress(&found, HIP_SYMBOL(scratch));
        if (status != hipSuccess || found == nullptr) {
            return hipFailure(status != hipSuccess ? status : hipErrorInvalidSymbol,
                              "hipGetSymbolAddress(scratch)", __FILE__, __LINE__);
        }
        cached = found;
    }
    *address = cached;
    return ZCGVS_OK;
}

}  // namespace

int prepareStaticScratch() {
    void* address = nullptr;
    return scratchAddress(&address);
}

}  // namespace zcgvs_hip

using namespace zcgvs_hip;

extern "C" {

std::size_t zcgvs_search_workspace_bytes(const zcgvs_search_desc* desc) {
    if (desc == nullptr) {
        setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: descriptor must not be null");
        return 0;
    }
    const Plan plan = makePlan(*desc);
    if (plan.status != ZCGVS_OK) {
        setError(plan.status, plan.error);
        return 0;
    }
    clearError();
    return plan.total;
}

int zcgvs_search_overflow_flags(const zcgvs_search_desc* desc, void* d_workspace,
                                std::uint32_t** d_flags) {
    if (desc == nullptr || d_flags == nullptr || d_workspace == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: null argument");
    }
    const Plan plan = makePlan(*desc);
    if (plan.status != ZCGVS_OK) {
        return setError(plan.status, plan.error);
    }
    *d_flags = reinterpret_cast<std::uint32_t*>(static_cast<std::uint8_t*>(d_workspace) + plan.overflow);
    return clearError();
}

int zcgvs_search_sketch_state(const zcgvs_search_desc* desc, void* d_workspace, float** d_slot_scores, int* slots,
                              int* rank, int* width, std::uint64_t** d_tau, std::uint64_t** d_tau_safe) {
    if (desc == nullptr || d_workspace == nullptr || d_slot_scores == nullptr || slots == nullptr ||
        rank == nullptr || width == nullptr || d_tau == nullptr || d_tau_safe == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: null argument");
    }
    const Plan plan = makePlan(*desc);
    if (plan.status != ZCGVS_OK) {
        return setError(plan.status, plan.error);
    }
    std::uint8_t* ws = static_cast<std::uint8_t*>(d_workspace);
    *width = plan.width;
    *slots = plan.sketch ? plan.sketch_slots : 0;
    *rank = plan.sketch ? plan.sketch_rank : 0;
    *d_slot_scores = plan.sketch ? reinterpret_cast<float*>(ws + plan.sketchbuf) : nullptr;
    *d_tau = plan.sketch ? reinterpret_cast<std::uint64_t*>(ws + plan.tau) : nullptr;
    *d_tau_safe = plan.sketch ? reinterpret_cast<std::uint64_t*>(ws + plan.tau_safe) : nullptr;
    return clearError();
}

namespace {

int searchTopk(const zcgvs_search_desc* desc, void* d_workspace, std::size_t workspace_bytes,
               int* d_out_indices, float* d_out_values, zcgvs_stream_t stream,
               zcgvs_event_t* events, int max_phases, int* phases_out) {
    if (desc == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: descriptor must not be null");
    }
    const zcgvs_search_desc& d = *desc;
    const Plan plan = makePlan(d);
    if (plan.status != ZCGVS_OK) {
        return setError(plan.status, plan.error);
    }
    if (d_workspace == nullptr || workspace_bytes < plan.total) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT,
                        "zcgvs: workspace of " + std::to_string(workspace_bytes) +
                            " bytes is smaller than the " + std::to_string(plan.total) + " needed");
    }
    if (d_out_indices == nullptr || d_out_values == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: output pointers must not be null");
    }
    std::uint8_t* ws = static_cast<std::uint8_t*>(d_workspace);
    const hipStream_t s = toStream(stream);
    const int batch = d.batch;
    const int dim = d.corpus.dim;
    int status = ZCGVS_OK;

    // 1. queries
    if (plan.binary) {
        status = zcgvs_launch_pack_binary(d.queries, ws + plan.qbits, batch, dim, stream);
    } else if (plan.per_vector) {
        status = launchQuantizeRows(d.queries, batch, dim, at<std::int8_t>(ws, plan.qi8),
                                    at<float>(ws, plan.qscale), s);
    }
    if (status != ZCGVS_OK) {
        return status;
    }

    if (plan.materialized) {
        if (phases_out != nullptr) {
            *phases_out = 0;
        }
        // the materialized pipeline never overflows; its flags are simply cleared
        zeroWordsKernel<<<1, 256, 0, s>>>(at<std::uint32_t>(ws, plan.overflow), static_cast<std::size_t>(batch));
        ZCGVS_LAUNCH_CHECK("zero flags");
        status = runMaterialized(d, plan, ws, d_out_indices, d_out_values, s);
        return status == ZCGVS_OK ? clearError() : status;
    }

    // 2. lexical scores (timed by the event pair after the scan phases' pairs, when there is one)
    if (plan.hybrid) {
        const int lex_pair = static_cast<int>(plan.phases.size());
        const bool timed = events != nullptr && lex_pair < max_phases;
        if (timed) {
            ZCGVS_HIP_RETURN(hipEventRecord(reinterpret_cast<hipEvent_t>(events[2 * lex_pair]), s));
        }
        status = launchLexicalScores(d.lex_offsets, d.lex_docs, d.lex_weights, d.lex_vocab_size, d.query_terms,
                                     d.lexical_stride, batch, static_cast<int>(d.corpus.doc_count),
                                     at<float>(ws, plan.lex), at<float>(ws, plan.lexmax),
                                     plan.lex_sorted ? at<std::int64_t>(ws, plan.lexbounds) : nullptr,
                                     d.lex_slice_table, d.lex_doc_count, s);
        if (status != ZCGVS_OK) {
            return status;
        }
        if (timed) {
            ZCGVS_HIP_RETURN(hipEventRecord(reinterpret_cast<hipEvent_t>(events[2 * lex_pair + 1]), s));
        }
    }

    // 3. phased scan + merge
    if (plan.use_mfma) {
        const long long n = d.corpus.doc_count;
        const long long padded = (n + kMfmaBlockRows - 1) / kMfmaBlockRows * kMfmaBlockRows;
        if (plan.direct_scales) {
            // the padded scales of a partial last tile (none when the corpus fills whole tiles)
            if (padded != n) {
                mergeMaskedScalesKernel<<<1, kMfmaBlockRows, 0, s>>>(d.corpus.row_scales, nullptr, n,
                                                                     padded - kMfmaBlockRows, kMfmaBlockRows,
                                                                     at<float>(ws, plan.mscales));
            }
        } else {
            mergeMaskedScalesKernel<<<static_cast<unsigned>(std::min<long long>(8192, (padded + 255) / 256)), 256, 0, s>>>(
                d.corpus.row_scales, d.mask, n, 0, padded, at<float>(ws, plan.mscales));
        }
        ZCGVS_LAUNCH_CHECK("merge mask");
    }
    std::uint64_t* keys = at<std::uint64_t>(ws, plan.keys);
    std::uint32_t* overflow = at<std::uint32_t>(ws, plan.overflow);
    // The exact fallback of a phased scan: a plan whose scan kernel reruns flagged queries runs
    // it after the scan (step 4); any other plan runs it in the launch of its last merge.
    const bool force = (d.flags & ZCGVS_SEARCH_FORCE_EXACT_PASS) != 0;
    const bool fuse_recovery = plan.recover && !plan.single_pass && !(plan.rerun && plan.phases.size() > 1 && !force);
    if (plan.single_pass) {
        if (phases_out != nullptr) {
            *phases_out = 1;
        }
        const bool timed = events != nullptr && max_phases > 0;
        if (timed) {
            ZCGVS_HIP_RETURN(hipEventRecord(reinterpret_cast<hipEvent_t>(events[0]), s));
        }
        SinglePassArgs single;
        single.width = plan.width;
        single.workgroups = plan.workgroups;
        single.cap = plan.sp_cap;
        single.groups = plan.sp_groups;
        single.seg = at<std::uint64_t>(ws, plan.seg);
        single.seg_count = at<std::uint32_t>(ws, plan.segcnt);
        single.seg_log2 = plan.seg_log2;
        status = launchSinglePass(recoverArgsOf(d, plan, ws), single, s);
        if (status != ZCGVS_OK) {
            return status;
        }
        if (timed) {
            ZCGVS_HIP_RETURN(hipEventRecord(reinterpret_cast<hipEvent_t>(events[1]), s));
        }
        MergeInputs in;
        in.seg = single.seg;
        in.seg_count = single.seg_count;
        in.n_seg = plan.segments / plan.sp_groups;
        in.seg_log2 = plan.seg_log2;
        if (plan.sp_groups > 1) {
            // Every (query, group) pair's top-width, then the results of up to 8 neighbouring
            // groups at a time (contiguous in the buffer: pair (q, g) at (q * groups + g) * width)
            // until one remains per query; each merge gathers at most 8192 keys in LDS.
            std::uint64_t* level[2] = {at<std::uint64_t>(ws, plan.sp_level),
                                       at<std::uint64_t>(ws, plan.sp_level) +
                                           static_cast<std::size_t>(batch) * plan.sp_groups * plan.width};
            status = launchSelectMerge(in, plan.width, batch * plan.sp_groups, level[0], nullptr, nullptr, nullptr,
                                       nullptr, s);
            if (status != ZCGVS_OK) {
                return status;
            }
            int groups = plan.sp_groups;
            int cur = 0;
            while (true) {
                const int fold = std::min(8, groups);
                in = MergeInputs{};
                in.dense = level[cur];
                in.n_dense = static_cast<long long>(fold) * plan.width;
                in.dense_stride = in.n_dense;
                groups /= fold;
                if (groups == 1) {
                    break;  // the last merge, below, writes the keys and the result
                }
                status = launchSelectMerge(in, plan.width, batch * groups, level[cur ^ 1], nullptr, nullptr, nullptr,
                                           nullptr, s);
                if (status != ZCGVS_OK) {
                    return status;
                }
                cur ^= 1;
            }
        }
        in.reset_overflow = true;  // (segments hold at most width keys: the flags end cleared)
        if (plan.sp_groups == 1 && plan.width <= kSortedSelectMaxK && in.n_seg <= kSortedMergeMaxSegments) {
            // each workgroup's list is sorted (single_pass.hip): the merge reads at most width
            // segments past their first key
            status = launchSortedSegmentMerge(in, plan.width, batch, keys, overflow,
                                              plan.rescore ? nullptr : d_out_indices,
                                              plan.rescore ? nullptr : d_out_values, s);
        } else {
            status = launchSelectMerge(in, plan.width, batch, keys, nullptr, overflow,
                                       plan.rescore ? nullptr : d_out_indices,
                                       plan.rescore ? nullptr : d_out_values, s);
        }
        if (status != ZCGVS_OK) {
            return status;
        }
    } else {
        const ScanArgs scan = scanArgsOf(d, plan, ws);
        if ((plan.use_mfma && !mfmaSupported(scan)) || (plan.use_mfma_float && !mfmaFloatSupported(scan)) ||
            (plan.use_mfma_binary && !mfmaBinarySupported(scan))) {
            return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: corpus or queries are not 16-byte aligned");
        }
        EmitArgs emit;
        emit.tau = at<std::uint64_t>(ws, plan.tau);
        emit.dense = at<std::uint64_t>(ws, plan.dense);
        emit.dense_stride = plan.dense_stride;
        emit.seg = plan.phases.size() > 1 ? at<std::uint64_t>(ws, plan.seg) : nullptr;
        emit.seg_count = plan.phases.size() > 1 ? at<std::uint32_t>(ws, plan.segcnt) : nullptr;
        emit.seg_log2 = plan.seg_log2;
        if (plan.sketch) {
            emit.sketch = at<float>(ws, plan.sketchbuf);
        }
        std::uint64_t* tau = at<std::uint64_t>(ws, plan.tau);
        std::uint32_t* flag_list = at<std::uint32_t>(ws, plan.flag_list);
        std::uint32_t* flag_count = at<std::uint32_t>(ws, plan.flag_count);

        if (phases_out != nullptr) {
            *phases_out = static_cast<int>(plan.phases.size());
        }
        // Without a rerun, the exact fallback runs in the launch of the last merge (one block per
        // query merges and, when it flags the query, recomputes its selection).
        RecoverArgs fused_recovery;
        if (fuse_recovery) {
            fused_recovery.force = force || plan.phases.size() <= 1;
            fused_recovery.width = plan.width;
            fused_recovery.out_keys = keys;
            fused_recovery.out_index = plan.rescore ? nullptr : d_out_indices;
            fused_recovery.out_score = plan.rescore ? nullptr : d_out_values;
        }
        for (std::size_t p = 0; p < plan.phases.size(); ++p) {
            const PhaseArgs& phase = plan.phases[p];
            const bool timed = events != nullptr && static_cast<int>(p) < max_phases;
            if (timed) {
                ZCGVS_HIP_RETURN(hipEventRecord(reinterpret_cast<hipEvent_t>(events[2 * p]), s));
            }
            if (plan.use_mfma) {
                status = launchMfmaScan(scan, phase, emit, plan.workgroups, s);
            } else if (plan.use_mfma_float) {
                status = launchMfmaFloatScan(scan, phase, emit, plan.workgroups, s);
            } else if (plan.use_mfma_binary) {
                status = launchMfmaBinaryScan(scan, phase, emit, plan.workgroups, s);
            } else {
                status = launchValuScan(scan, phase, emit, plan.workgroups, s);
            }
            if (status != ZCGVS_OK) {
                return status;
            }
            if (timed) {
                ZCGVS_HIP_RETURN(hipEventRecord(reinterpret_cast<hipEvent_t>(events[2 * p + 1]), s));
            }
            const bool last = p + 1 == plan.phases.size();
            if (phase.sketch) {
                // the speculative threshold and the guaranteed one; clears the flagged list
                status = launchSketchThreshold(emit.sketch, plan.sketch_slots, batch, plan.sketch_rank, plan.width,
                                               tau, at<std::uint64_t>(ws, plan.tau_safe), flag_count, s);
                if (status != ZCGVS_OK) {
                    return status;
                }
                continue;
            }
            MergeInputs in;
            if (plan.sketch) {
                // the one merge of the speculative scan
                in.seg = emit.seg;
                in.seg_count = emit.seg_count;
                in.n_seg = plan.segments;
                in.seg_log2 = plan.seg_log2;
                in.reset_overflow = true;
                in.require_full = true;
                in.fallback_tau = at<std::uint64_t>(ws, plan.tau_safe);
            } else if (p == 0) {
                in.dense = emit.dense;
                in.n_dense = phase.items * phase.block_rows;
                in.dense_stride = plan.dense_stride;
                in.reset_overflow = true;
                in.zero_count = flag_count;
            } else {
                in.prev = keys;
                in.k_prev = plan.width;
                in.seg = emit.seg;
                in.seg_count = emit.seg_count;
                in.n_seg = plan.segments;
                in.seg_log2 = plan.seg_log2;
            }
            if (last) {
                in.final_merge = true;
                in.flag_list = flag_list;
                in.flag_count = flag_count;
                in.rerun_tau = tau;
            }
            const bool write_out = last && !plan.rescore;
            if (last && fuse_recovery) {
                status = launchMergeRecover(in, plan.width, batch, keys, overflow, write_out ? d_out_indices : nullptr,
                                            write_out ? d_out_values : nullptr, recoverArgsOf(d, plan, ws),
                                            fused_recovery, s);
            } else {
                status = launchSelectMerge(in, plan.width, batch, keys, last ? nullptr : tau, overflow,
                                           write_out ? d_out_indices : nullptr,
                                           write_out ? d_out_values : nullptr, s);
            }
            if (status != ZCGVS_OK) {
                return status;
            }
        }
    }

    // 4. the exact fallback for the flagged queries of a rerun plan (near-empty launches
    //    otherwise): the scan kernel's rerun over the whole corpus, then the selection from the
    //    rerun's segments, or the last resort's recomputation (other plans ran it with the last
    //    merge)
    if (plan.recover && !fuse_recovery) {
        const bool multi_phase = plan.phases.size() > 1;
        const bool rerun = plan.rerun && multi_phase && !force;
        RecoverArgs recovery;
        recovery.flags = overflow;
        recovery.force = force || !multi_phase;
        recovery.width = plan.width;
        recovery.out_keys = keys;
        recovery.out_index = plan.rescore ? nullptr : d_out_indices;
        recovery.out_score = plan.rescore ? nullptr : d_out_values;
        recovery.flag_list = at<std::uint32_t>(ws, plan.flag_list);
        recovery.flag_count = at<std::uint32_t>(ws, plan.flag_count);
        if (rerun) {
            EmitArgs again;
            again.tau = at<std::uint64_t>(ws, plan.tau);
            again.seg = at<std::uint64_t>(ws, plan.seg);
            again.seg_count = at<std::uint32_t>(ws, plan.segcnt);
            again.seg_log2 = plan.rerun_seg_log2;
            again.q_list = recovery.flag_list;
            again.q_list_count = recovery.flag_count;
            const ScanArgs scan = scanArgsOf(d, plan, ws);
            status = plan.use_mfma ? launchMfmaScan(scan, plan.full, again, plan.workgroups, s)
                                   : launchMfmaBinaryScan(scan, plan.full, again, plan.workgroups, s);
            if (status != ZCGVS_OK) {
                return status;
            }
            recovery.seg = again.seg;
            recovery.seg_count = again.seg_count;
            recovery.n_seg = plan.segments;
            recovery.seg_log2 = plan.rerun_seg_log2;
        }
        status = launchRecover(recoverArgsOf(d, plan, ws), recovery, s);
        if (status != ZCGVS_OK) {
            return status;
        }
    }

    // 5. rescore
    if (plan.rescore) {
        std::uint64_t* rescored = at<std::uint64_t>(ws, plan.rescored);
        status = launchRescoreKeys(d.rescore.data, d.rescore.dtype, d.rescore.scale,
                                   static_cast<int>(std::min<std::int64_t>(d.rescore.doc_count, INT32_MAX)),
                                   dim, d.queries, batch, keys, plan.width, d.metric, rescored, s);
        if (status != ZCGVS_OK) {
            return status;
        }
        MergeInputs in;
        in.dense = rescored;
        in.n_dense = plan.width;
        in.dense_stride = plan.width;
        status = launchSelectMerge(in, d.k, batch, keys, nullptr, nullptr, d_out_indices,
                                   d_out_values, s);
        if (status != ZCGVS_OK) {
            return status;
        }
    }
    return clearError();
}

}  // namespace

int zcgvs_search_topk(const zcgvs_search_desc* desc, void* d_workspace, std::size_t workspace_bytes,
                      int* d_out_indices, float* d_out_values, zcgvs_stream_t stream) {
    return searchTopk(desc, d_workspace, workspace_bytes, d_out_indices, d_out_values, stream,
                      nullptr, 0, nullptr);
}

int zcgvs_search_topk_profiled(const zcgvs_search_desc* desc, void* d_workspace,
                               std::size_t workspace_bytes, int* d_out_indices,
                               float* d_out_values, zcgvs_stream_t stream, zcgvs_event_t* events,
                               int max_phases, int* phases) {
    return searchTopk(desc, d_workspace, workspace_bytes, d_out_indices, d_out_values, stream,
                      events, max_phases, phases);
}

int zcgvs_search_phase_rows(const zcgvs_search_desc* desc, long long* rows, int max_phases,
                            int* phases) {
    if (desc == nullptr || phases == nullptr || (rows == nullptr && max_phases > 0)) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: descriptor and outputs must not be null");
    }
    const Plan plan = makePlan(*desc);
    if (plan.status != ZCGVS_OK) {
        return setError(plan.status, plan.error);
    }
    *phases = static_cast<int>(plan.phases.size());
    const long long n = desc->corpus.doc_count;
    const long long last_block = (n + plan.block_rows - 1) / plan.block_rows - 1;
    for (std::size_t p = 0; p < plan.phases.size() && static_cast<int>(p) < max_phases; ++p) {
        const PhaseArgs& phase = plan.phases[p];
        long long r = phase.items * phase.block_rows;
        // the partial last block belongs to the phase whose stride divides it and skip does not
        const bool holds_last = last_block % phase.stride == 0 &&
                                (phase.skip == 0 || last_block % (phase.stride * phase.skip) != 0);
        if (holds_last) {
            r -= (last_block + 1) * plan.block_rows - n;
        }
        rows[p] = r;
    }
    return clearError();
}

std::size_t zcgvs_static_scratch_bytes(void) { return kStaticScratchBytes; }

int zcgvs_search_topk_noalloc(const zcgvs_search_desc* desc, int* d_out_indices, float* d_out_values,
                              zcgvs_stream_t stream) {
    if (desc == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: descriptor must not be null");
    }
    const Plan plan = makePlan(*desc);
    if (plan.status != ZCGVS_OK) {
        return setError(plan.status, plan.error);
    }
    if (plan.total > kStaticScratchBytes) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT,
                        "zcgvs: this search needs " + std::to_string(plan.total) +
                            " bytes of workspace, more than the " + std::to_string(kStaticScratchBytes) +
                            "-byte static scratch of zcgvs_search_topk_noalloc; pass a workspace to "
                            "zcgvs_search_topk instead");
    }
    void* address = nullptr;
    const int status = scratchAddress(&address);
    if (status != ZCGVS_OK) {
        return status;
    }
    return searchTopk(desc, address, kStaticScratchBytes, d_out_indices, d_out_values, stream, nullptr, 0,
                      nullptr);
}

}  // extern "C"
