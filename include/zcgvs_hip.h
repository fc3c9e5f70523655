/*
 * zcgvs_hip.h - C ABI of the MI355X (gfx950) zero-copy search hot path.
 *
 * Every entry point takes plain device pointers, sizes and a stream handle and returns a
 * zcgvs_status code. Nothing here throws, and no C++ or torch type crosses the boundary.
 * The message describing the most recent failure on the calling thread is returned by
 * zcgvs_last_error().
 *
 * Error contract (mirrors the reference's exception split, include/zcgvs/core/cuda_check.hpp
 * and src/search/searcher.cpp:91-135):
 *   ZCGVS_ERR_INVALID_ARGUMENT  - the reference throws std::invalid_argument;
 *   ZCGVS_ERR_RUNTIME           - the reference throws std::runtime_error (e.g. N > INT32_MAX);
 *   ZCGVS_ERR_HIP               - a HIP runtime call failed (the reference's CudaError).
 * Launchers that receive empty work (count <= 0) return ZCGVS_OK without launching, exactly
 * like the reference launchers (src/cuda/similarity.cu:356-358, topk.cu:143-145).
 *
 * Launchers are asynchronous on the given stream, never allocate device memory, never
 * synchronize, and are safe to record into a HIP graph (zcgvs_graph_begin_capture). The one
 * exception is zcgvs_memset, which must not be recorded into a graph; use zcgvs_fill_u32.
 *
 * Enumerations keep the reference's numeric codes, which are part of its on-disk format:
 *   metric (include/zcgvs/core/metric.hpp:8-12), dtype (include/zcgvs/core/scalar_type.hpp:12-17).
 *
 * Top-k ordering (all selection entry points): score descending, ties broken by the lower
 * corpus index, i.e. the order std::stable_sort gives in tests/cpp/cpu_reference.hpp:26-34.
 * -0.0f ranks equal to +0.0f; a NaN score ranks below every other score.
 */
#ifndef ZCGVS_HIP_H
#define ZCGVS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------------------------
 * Status, enums, opaque handles
 * ---------------------------------------------------------------------------------------- */
enum zcgvs_status {
    ZCGVS_OK = 0,
    ZCGVS_ERR_INVALID_ARGUMENT = 1,
    ZCGVS_ERR_RUNTIME = 2,
    ZCGVS_ERR_HIP = 3,
    ZCGVS_ERR_UNSUPPORTED = 4
};

/* include/zcgvs/core/metric.hpp:8-12 */
enum zcgvs_metric { ZCGVS_METRIC_COSINE = 0, ZCGVS_METRIC_DOT = 1, ZCGVS_METRIC_L2 = 2 };

/* include/zcgvs/core/scalar_type.hpp:12-17 */
enum zcgvs_dtype {
    ZCGVS_DTYPE_F32 = 0,
    ZCGVS_DTYPE_F16 = 1,
    ZCGVS_DTYPE_I8 = 2,
    ZCGVS_DTYPE_BINARY = 3
};

/* How an int8 corpus is scored.
 *  REFERENCE: (int8 * one matrix-wide scale) against a float32 query, accumulated in float32,
 *             as src/cuda/similarity.cu:59-67 and include/zcgvs/cuda/decode.cuh:24-26 do.
 *  PER_VECTOR: each row r carries its own scale s_r = max|x_r| / 127; queries are quantized the
 *             same way on the device; score = (float)(int32 dot) * (s_q * s_r), evaluated in
 *             exactly that order. No counterpart in the reference (its format has one scale). */
enum zcgvs_int8_mode { ZCGVS_INT8_REFERENCE = 0, ZCGVS_INT8_PER_VECTOR = 1 };

typedef void* zcgvs_stream_t; /* hipStream_t; NULL is the null stream   */
typedef void* zcgvs_event_t;  /* hipEvent_t                               */
typedef void* zcgvs_graph_t;  /* hipGraphExec_t (instantiated graph)      */

/* Message for the most recent non-OK status returned on this thread ("" if none). */
const char* zcgvs_last_error(void);
/* Library version string, e.g. "zcgvs-hip 0.1.0 gfx950". */
const char* zcgvs_version(void);

/* ------------------------------------------------------------------------------------------
 * Device, memory, streams, events, graphs - the thin runtime layer the C++17 host uses in
 * place of include/zcgvs/core/{cuda_context,device_buffer,pinned_buffer,cuda_stream}.hpp.
 * ---------------------------------------------------------------------------------------- */
typedef struct zcgvs_device_info {
    char name[256];
    char arch[64];             /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    size_t total_memory;       /* bytes */
    int compute_units;
    int clock_khz;
    int memory_clock_khz;
    int memory_bus_width;      /* bits */
    int l2_cache_bytes;
    int major;
    int minor;
    /* 2 * memory clock * bus width / 8, the formula of include/zcgvs/core/cuda_context.hpp:20-23 */
    double peak_bandwidth_gbs;
} zcgvs_device_info;

int zcgvs_device_count(int* count);
int zcgvs_set_device(int device);                       /* src/core/cuda_context.cpp:9 */
int zcgvs_get_device(int* device);
int zcgvs_device_query(int device, zcgvs_device_info* out); /* src/core/cuda_context.cpp:23-45 */
int zcgvs_device_synchronize(void);

/* Measured HBM rates of the current device, the achievable counterpart of peak_bandwidth_gbs
 * (the reference derives only that nominal peak, include/zcgvs/core/cuda_context.hpp:20-23, and
 * prints each scan's GB/s against it, apps/bench_kernels.cu:133-143). A streaming read and a
 * streaming copy over two `bytes`-byte buffers (at least 64 MiB; use several times the 256 MiB
 * last-level cache) are each timed `iterations` times at a few grid sizes; the best launch gives
 * *read_gbs (bytes read per second) and *copy_gbs (bytes read + written per second), in 1e9
 * bytes/s. Allocates, frees and synchronizes: never call it inside a graph capture. */
int zcgvs_measure_hbm_bandwidth(size_t bytes, int iterations, double* read_gbs, double* copy_gbs);

int zcgvs_malloc(void** ptr, size_t bytes);           /* device_buffer.hpp:40-56 */
int zcgvs_free(void* ptr);
int zcgvs_host_alloc(void** ptr, size_t bytes);       /* pinned_buffer.hpp:14-67 */
int zcgvs_host_free(void* ptr);
int zcgvs_memcpy_h2d(void* dst, const void* src, size_t bytes, zcgvs_stream_t stream);
int zcgvs_memcpy_d2h(void* dst, const void* src, size_t bytes, zcgvs_stream_t stream);
int zcgvs_memcpy_d2d(void* dst, const void* src, size_t bytes, zcgvs_stream_t stream);
/* Not graph-capture safe (records a memset node); use zcgvs_fill_u32 inside captures. */
int zcgvs_memset(void* dst, int value, size_t bytes, zcgvs_stream_t stream);
/* Fills `count` 32-bit words with `value` using a kernel (capture safe). */
int zcgvs_fill_u32(void* dst, uint32_t value, size_t count, zcgvs_stream_t stream);

int zcgvs_stream_create(zcgvs_stream_t* stream);      /* cuda_stream.hpp:9-43 */
int zcgvs_stream_destroy(zcgvs_stream_t stream);
int zcgvs_stream_synchronize(zcgvs_stream_t stream);

int zcgvs_event_create(zcgvs_event_t* event);
int zcgvs_event_destroy(zcgvs_event_t event);
int zcgvs_event_record(zcgvs_event_t event, zcgvs_stream_t stream);
int zcgvs_event_synchronize(zcgvs_event_t event);
int zcgvs_event_elapsed_ms(float* ms, zcgvs_event_t start, zcgvs_event_t end);

/* Stream capture into an instantiated graph (src/search/searcher.cpp:305-342). Capture uses
 * the thread-local mode. end_capture instantiates and returns the executable graph. */
int zcgvs_graph_begin_capture(zcgvs_stream_t stream);
int zcgvs_graph_end_capture(zcgvs_stream_t stream, zcgvs_graph_t* graph);
int zcgvs_graph_launch(zcgvs_graph_t graph, zcgvs_stream_t stream);
int zcgvs_graph_destroy(zcgvs_graph_t graph);

/* ------------------------------------------------------------------------------------------
 * Kernel launchers. Each one replaces the reference launcher named in its comment, with the
 * same argument order and meaning, a HIP stream in place of the CUDA stream, and a status code
 * in place of exceptions.
 * ---------------------------------------------------------------------------------------- */

/* src/cuda/similarity.cu:345-398 launchSimilarity.
 * d_scores[q * doc_count + doc] = score of query q against document doc.
 * d_queries: [batch, dim] float32, or [batch, ceil(dim/32)] packed uint32 words for a BINARY
 * corpus (bit b of word w = dimension 32w+b, set iff value >= 0). Masked documents (mask byte 0)
 * score -FLT_MAX. Cosine is a raw dot product (inputs are assumed L2-normalized). L2 scores are
 * the negated squared distance. Binary scores are (dim - 2*hamming) / dim. Unmasked cosine/dot
 * batches of at least 4 float32/float16 queries with dim 128, 256, 384 or 512 are computed on the
 * matrix cores (float32 products and sums in another order: equal to the scalar loop within
 * float32 rounding). */
int zcgvs_launch_similarity(const void* d_corpus, int dtype, float scale, int doc_count, int dim,
                            const void* d_queries, int batch, const uint8_t* d_mask, int metric,
                            float* d_scores, zcgvs_stream_t stream);

/* Same contract as zcgvs_launch_similarity for an int8 corpus in ZCGVS_INT8_PER_VECTOR mode:
 * d_corpus [doc_count, dim] int8 with d_row_scales [doc_count]; d_queries [batch, dim] int8 with
 * d_query_scales [batch]. Metric must be COSINE or DOT. No reference counterpart. Scores are
 * (float)(int32 dot) * (s_q * s_r) on every path (unmasked batches of at least 8 queries over a
 * whole number of 64-row tiles with dim 256-1024 run on the matrix cores). */
int zcgvs_launch_similarity_i8i8(const int8_t* d_corpus, const float* d_row_scales,
                                 int doc_count, int dim, const int8_t* d_queries,
                                 const float* d_query_scales, int batch, const uint8_t* d_mask,
                                 int metric, float* d_scores, zcgvs_stream_t stream);

int zcgvs_similarity_query_tile(void);                                /* similarity.cu:309 */
size_t zcgvs_similarity_shared_bytes(int dtype, int dim, int batch);  /* similarity.cu:337-343 */

/* src/cuda/topk.cu:112-130 sizing helpers. zcgvs_topk_scratch_elements is the per-query element
 * count of EACH of the four scratch buffers zcgvs_launch_topk takes. */
int zcgvs_topk_tile_size(void);
int zcgvs_topk_merge_tile(void);
int zcgvs_topk_max_k(void);
int zcgvs_topk_block_count(int doc_count);
int zcgvs_topk_scratch_elements(int doc_count, int k);

/* src/cuda/topk.cu:132-189 launchTopK. Selects the k best of each [batch, doc_count] score row,
 * descending, lowest index first on equal scores. Scratch buffers are each
 * batch * zcgvs_topk_scratch_elements(doc_count, k) elements. k <= zcgvs_topk_max_k() and
 * k <= doc_count or ZCGVS_ERR_INVALID_ARGUMENT. */
int zcgvs_launch_topk(const float* d_scores, int doc_count, int k, int batch, int* d_out_indices,
                      float* d_out_values, float* d_scratch_values_a, int* d_scratch_indices_a,
                      float* d_scratch_values_b, int* d_scratch_indices_b,
                      zcgvs_stream_t stream);

/* src/cuda/rescore.cu:83-130 launchGatherRescore / rescoreSharedBytes.
 * d_values[q * C + slot] = exact score of corpus row d_candidate_indices[q * C + slot] against
 * float32 query q; an index < 0 or >= doc_count gives -FLT_MAX. BINARY storage is rejected. */
size_t zcgvs_rescore_shared_bytes(int dim);
int zcgvs_launch_gather_rescore(const void* d_corpus, int dtype, float scale, int doc_count,
                                int dim, const float* d_queries, int batch,
                                const int* d_candidate_indices, int candidate_count, int metric,
                                float* d_values, zcgvs_stream_t stream);

/* src/cuda/rescore.cu:132-146 launchRemapIndices. */
int zcgvs_launch_remap_indices(const int* d_candidate_indices, const int* d_local_indices,
                               int candidate_count, int k, int batch, int* d_out_indices,
                               zcgvs_stream_t stream);

/* src/cuda/lexical.cu:78-92 launchBm25. Scatter-adds the posting weights of the query's terms
 * into d_scores (zeroed by the caller). Terms < 0 are skipped, as are documents outside
 * [0, doc_count); term ids must be below the index's vocabulary size, as in the reference.
 * Terms are accumulated in slot order, so every document's sum is formed in the same order on
 * every run. */
int zcgvs_launch_bm25(const int64_t* d_offsets, const int* d_docs, const float* d_weights,
                      const int* d_query_terms, int term_count, int doc_count, float* d_scores,
                      zcgvs_stream_t stream);

/* Batched form of zcgvs_launch_bm25: d_query_terms [batch, term_stride], d_scores
 * [batch, doc_count] (zeroed by the caller). One launch per term slot instead of one per
 * (query, slot) as src/search/searcher.cpp:241-249 does. */
int zcgvs_launch_bm25_batched(const int64_t* d_offsets, const int* d_docs,
                              const float* d_weights, const int* d_query_terms, int term_stride,
                              int batch, int doc_count, float* d_scores, zcgvs_stream_t stream);

/* Slice table of a lexical index whose postings ascend strictly by document (the
 * ZCGVS_SEARCH_SORTED_POSTINGS layout): d_table[t * S + c] = the number of term t's postings whose
 * document is below c * 4096 for c < S - 1, and below doc_count for c = S - 1, with
 * S = ceil(doc_count / 4096) + 1 (doc_count <= 2^31 - 1). Built once per index (one binary search
 * per entry), it lets every hybrid search take its terms' 4096-document slice bounds from the
 * table (zcgvs_search_desc.lex_slice_table). No reference counterpart: the reference's BM25
 * (src/cuda/lexical.cu:17-42) scatters every posting with atomics and keeps no such table.
 * zcgvs_lexical_slice_table_bytes returns 0 for an empty index or too many documents. */
size_t zcgvs_lexical_slice_table_bytes(int vocab_size, int64_t doc_count);
int zcgvs_build_lexical_slice_table(const int64_t* d_offsets, const int* d_docs, int vocab_size,
                                    int64_t doc_count, uint32_t* d_table, zcgvs_stream_t stream);

/* src/cuda/lexical.cu:94-105 launchMaxPositive: *d_max = max(*d_max, max_i values[i]) for
 * values >= 0 (caller zeroes *d_max). */
int zcgvs_launch_max_positive(const float* d_values, int count, float* d_max,
                              zcgvs_stream_t stream);

/* src/cuda/lexical.cu:107-123 launchFuseScores, in place:
 * dense[i] = weight * dense[i] + (1 - weight) * lexical[i] * (max > 0 ? 1/max : 0). */
int zcgvs_launch_fuse_scores(float* d_dense, const float* d_lexical, const float* d_lexical_max,
                             float weight, int count, zcgvs_stream_t stream);

/* src/cuda/convert.cu:55-93 launchConvertF32ToF16 / launchConvertF32ToI8 / launchPackBinary. */
int zcgvs_launch_convert_f32_to_f16(const float* d_src, void* d_dst_half, size_t count,
                                    zcgvs_stream_t stream);
int zcgvs_launch_convert_f32_to_i8(const float* d_src, void* d_dst_int8, size_t count,
                                   float scale, zcgvs_stream_t stream);
int zcgvs_launch_pack_binary(const float* d_src, void* d_dst_words, int rows, int dim,
                             zcgvs_stream_t stream);

/* Per-row symmetric int8 quantization (ZCGVS_INT8_PER_VECTOR): for every row,
 * s = max|x| / 127 (1.0 for an all-zero row), q = clamp(rint(x * (1/s)), -127, 127).
 * No reference counterpart; the reciprocal rule is that of src/cuda/convert.cu:25-32. */
int zcgvs_launch_quantize_rows_i8(const float* d_src, int rows, int dim, int8_t* d_dst,
                                  float* d_scales, zcgvs_stream_t stream);

/* ------------------------------------------------------------------------------------------
 * Fused search: the whole device pipeline of src/search/searcher.cpp:209-285 (scan, optional
 * BM25 fusion, top-k, optional gather rescore + second top-k + remap) without a [batch, N]
 * score matrix. Only [batch, k] ids and scores are written.
 * ---------------------------------------------------------------------------------------- */
typedef struct zcgvs_store_desc {
    const void* data;          /* [doc_count, row_stride] device rows                         */
    int64_t doc_count;
    int dim;
    int dtype;                 /* enum zcgvs_dtype                                             */
    float scale;               /* matrix-wide int8 scale (ZCGVS_INT8_REFERENCE)               */
    const float* row_scales;   /* [doc_count] per-row int8 scales (ZCGVS_INT8_PER_VECTOR)     */
} zcgvs_store_desc;

typedef struct zcgvs_search_desc {
    zcgvs_store_desc corpus;   /* primary (scanned) store                                      */
    zcgvs_store_desc rescore;  /* rescore store; data == NULL disables the rescore stage        */
    const float* queries;      /* [batch, dim] float32 device queries                           */
    int batch;
    int k;                     /* final top-k, 1..zcgvs_topk_max_k()                            */
    int metric;                /* enum zcgvs_metric                                             */
    int int8_mode;             /* enum zcgvs_int8_mode (int8 corpus only)                       */
    const uint8_t* mask;       /* optional [doc_count] allow-mask                               */
    int rescore_candidates;    /* C; > 0 with rescore.data enables the rescore stage           */
    /* Hybrid lexical stage (src/search/searcher.cpp:235-259); enabled when query_terms != NULL
     * and lexical_stride > 0. */
    const int64_t* lex_offsets;
    const int* lex_docs;
    const float* lex_weights;
    int64_t lex_doc_count;
    int lex_vocab_size;        /* term ids >= this are skipped                                  */
    const int* query_terms;    /* [batch, lexical_stride] device term ids, -1 padded           */
    int lexical_stride;
    float dense_weight;
    int flags;                 /* zcgvs_search_flags bits; 0 for the default pipeline           */
    /* Optional slice table of the lexical index (zcgvs_build_lexical_slice_table over
     * lex_doc_count documents); with ZCGVS_SEARCH_SORTED_POSTINGS the BM25 stage reads its terms'
     * slice bounds from it instead of searching the postings. NULL: searched per call. */
    const uint32_t* lex_slice_table;
} zcgvs_search_desc;

/* zcgvs_search_desc.flags. ZCGVS_SEARCH_MATERIALIZE runs the reference-order pipeline (a
 * [batch, doc_count] score matrix in the workspace, then zcgvs_launch_topk) instead of the fused
 * scan; its workspace is correspondingly larger.
 * By default the BM25 stage scatters each query's postings term slot by term slot, which takes
 * postings in any order, like the reference's launchBm25 (src/cuda/lexical.cu:78-92).
 * ZCGVS_SEARCH_SORTED_POSTINGS states that every term's postings ascend strictly by document, one
 * per document (the layout the reference's index builder writes,
 * python/zcgvs_tools/build_lexical.py:147-163); the stage then reads them in document-range
 * slices instead, with no atomics and no clearing pass. Scores are bit-identical between the
 * two forms; with the flag set on postings that break the contract they are undefined.
 * ZCGVS_SEARCH_UNSORTED_POSTINGS names the default explicitly; setting it together with
 * ZCGVS_SEARCH_SORTED_POSTINGS is an invalid argument.
 * ZCGVS_SEARCH_FORCE_EXACT_PASS runs the exact device fallback (see zcgvs_search_topk) for every
 * query instead of only the ones whose candidate buffers overflowed; for tests and verification.
 * ZCGVS_SEARCH_TEST_TINY_SEGMENTS gives every candidate segment of the first attempt two slots, so
 * that almost every query overflows and takes the fallback through its overflow flag; for tests
 * only.
 * ZCGVS_SEARCH_TEST_HIGH_THRESHOLD sets the speculative threshold of a sketch-planned search (see
 * zcgvs_search_topk) to the best sampled score, so that most queries find fewer than k candidates
 * and take the fallback; for tests only (no effect on other plans).
 * ZCGVS_SEARCH_TEST_TINY_RERUN gives the rerun of flagged queries (sketch-planned and int8
 * matrix-core searches) segments of two slots per listed query when every query is listed, so
 * that, with ZCGVS_SEARCH_TEST_TINY_SEGMENTS listing almost every query, the reruns overflow too
 * and the last resort runs; for tests only. */
enum zcgvs_search_flags {
    ZCGVS_SEARCH_MATERIALIZE = 1,
    ZCGVS_SEARCH_UNSORTED_POSTINGS = 2,
    ZCGVS_SEARCH_SORTED_POSTINGS = 4,
    ZCGVS_SEARCH_FORCE_EXACT_PASS = 8,
    ZCGVS_SEARCH_TEST_TINY_SEGMENTS = 16,
    ZCGVS_SEARCH_TEST_HIGH_THRESHOLD = 32,
    ZCGVS_SEARCH_TEST_TINY_RERUN = 64
};

/* Bytes of device workspace zcgvs_search_topk needs for this descriptor (0 on error). */
size_t zcgvs_search_workspace_bytes(const zcgvs_search_desc* desc);

/* Runs the fused pipeline. d_out_indices/d_out_values are [batch, k]. The workspace must be
 * zcgvs_search_workspace_bytes(desc) bytes; its contents need no initialization. Capture safe.
 * The result is the exact top-k for every input: the scan keeps only candidates above a sampled
 * threshold in bounded per-workgroup buffers. A per-vector int8 search on the matrix cores, or a
 * binary search of 4 or more queries at 512 or 1024 bits, over a large corpus is sketch-planned: a first launch over
 * every 32nd block (64th for binary) records per slot (a row half of an int8 workgroup, a pair of a binary
 * workgroup's wavefronts) the best score of each query, and one scan of the whole corpus keeps
 * the keys at or above the j-th best of those scores (a threshold that is likely, not certain, to
 * lie below the k-th best key); other searches run threshold phases whose thresholds are certain
 * lower bounds. The search's last merge flags a query whose buffers overflowed (a corpus whose
 * best rows crowd into a few blocks) or which found fewer than k keys above a speculative
 * threshold; flagged queries are completed on the device, in the same call and stream, by the
 * exact fallback: for a sketch-planned search the scan runs once more over the whole corpus for
 * just those queries with a threshold that is a certain lower bound and the batch's candidate
 * buffers shared among them, and the selection is taken from that; for other scans, or when that
 * rerun overflows too, one workgroup per query selects over recomputed scores (a few corpus
 * reads).
 * zcgvs_search_overflow_flags tells which queries took the fallback. A search of at most four
 * queries selecting at most 1024 keys each (k, or rescore_candidates with a rescore store) that
 * no matrix-core scan takes reads the corpus in a single pass whose per-workgroup lists are exact
 * (selections above 32 keys merge groups of workgroups first); it never overflows.
 * Non-finite inputs: float32 rows of 256 or 384 dims searched with 32 to 128 queries per launch
 * are scanned on the bf16 matrix cores as exact three-part splits, where a row or query with an
 * infinite or NaN component scores NaN (it ranks last); every other scan follows the IEEE sum,
 * where such a score can be +inf and rank first. So with non-finite data the result can depend
 * on the batch size (the reference defines no order for non-finite scores either). */
int zcgvs_search_topk(const zcgvs_search_desc* desc, void* d_workspace, size_t workspace_bytes,
                      int* d_out_indices, float* d_out_values, zcgvs_stream_t stream);

/* No counterpart in the reference. For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): zcgvs_search_topk with
 * its workspace in a library-owned static device array of zcgvs_static_scratch_bytes() bytes
 * (64 MiB) per device instead of a caller's buffer. A search whose workspace
 * (zcgvs_search_workspace_bytes) exceeds that size is rejected with ZCGVS_ERR_INVALID_ARGUMENT;
 * nothing is allocated or freed, on the host's HIP side or the device. Every call on one device
 * shares that device's array: calls that overlap on one GPU (concurrent streams, threads) race
 * and must be serialized by the caller. The results equal zcgvs_search_topk's. The array's device
 * address is looked up on the first call on a device, or earlier by zcgvs_graph_begin_capture,
 * so a call recorded into a graph performs no lookup. */
size_t zcgvs_static_scratch_bytes(void);
int zcgvs_search_topk_noalloc(const zcgvs_search_desc* desc, int* d_out_indices, float* d_out_values,
                              zcgvs_stream_t stream);

/* Measurement hook: zcgvs_search_topk that also records events[2p] and events[2p + 1] on `stream`
 * immediately before and after the scan launches of phase p, for p < max_phases, and returns the
 * number of phases in *phases. A fused hybrid search also brackets its lexical (BM25) stage with
 * the next pair, events[2 * phases] and events[2 * phases + 1], when max_phases > *phases. The events must have been created with zcgvs_event_create. Not
 * meant for graph capture. No reference counterpart (the reference times the whole pipeline with
 * one event pair, src/search/searcher.cpp:358-365). */
int zcgvs_search_topk_profiled(const zcgvs_search_desc* desc, void* d_workspace,
                               size_t workspace_bytes, int* d_out_indices, float* d_out_values,
                               zcgvs_stream_t stream, zcgvs_event_t* events, int max_phases,
                               int* phases);

/* Corpus rows each scan phase of the fused pipeline visits for `desc` (rows[p] for p <
 * max_phases; the phase count in *phases; 0 phases when the pipeline materializes the score
 * matrix instead; one phase of doc_count rows for the single pass). Host only; used to price the
 * scan launches. No reference counterpart. */
int zcgvs_search_phase_rows(const zcgvs_search_desc* desc, long long* rows, int max_phases,
                            int* phases);

/* Device address of the [batch] uint32 overflow flags inside a workspace laid out for `desc`,
 * valid after the stream has completed the search: non-zero when that query's candidate buffers
 * overflowed and its result came from the exact device fallback (the result is exact either way;
 * the flags are for monitoring). */
int zcgvs_search_overflow_flags(const zcgvs_search_desc* desc, void* d_workspace,
                                uint32_t** d_flags);

/* Device addresses, inside a workspace laid out for `desc`, of a sketch-planned search's sketch
 * state, valid after the stream has completed the search: the slot scores (*slots x batch
 * float32, slot-major: the best score of each query over the slot's rows, -inf for a slot that
 * saw none) and two [batch] threshold keys (a key is kept when it is at least the threshold):
 * the speculative one, ordered32(the *rank-th best slot score) << 32 (for a flagged query the
 * merge replaces it by its rerun's threshold), and the certain one, of the *width-th best slot
 * score. A search that is not sketch-planned sets *slots and *rank to 0 and the addresses to
 * null. For monitoring and tests; no reference counterpart. */
int zcgvs_search_sketch_state(const zcgvs_search_desc* desc, void* d_workspace, float** d_slot_scores,
                              int* slots, int* rank, int* width, uint64_t** d_tau, uint64_t** d_tau_safe);

/* ------------------------------------------------------------------------------------------
 * Synthetic data on the device (benchmarks and large parity runs). Row r of a matrix generated
 * with `seed` depends only on (seed, r): a counter-based splitmix64 stream, Box-Muller in
 * double precision, rounded to float32, then L2-normalized in float32 in dimension order.
 * ---------------------------------------------------------------------------------------- */
int zcgvs_generate_normalized(float* d_out, int64_t rows, int dim, uint64_t seed,
                              int64_t row_offset, zcgvs_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* ZCGVS_HIP_H */
