/*
 * CPU oracle of the zero-copy search hot path - TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library,
 * and only to check or time against the HIP path; the product never calls it.
 *
 * Each function restates, in plain C, the semantics the reference fixes for one step of the
 * path (paths are relative to the reference repository). Build with -ffp-contract=off so every
 * float multiply and add rounds separately, as the reference's CPU loops do.
 *
 * Ordering used by every selection here: score descending, and the lower index first among
 * equal scores (std::stable_sort over ascending indices, tests/cpp/cpu_reference.hpp:26-34);
 * -0.0 compares equal to +0.0 and NaN ranks below every number.
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ZO_COSINE 0
#define ZO_DOT 1
#define ZO_L2 2

/* ---------------------------------------------------------------------------------------- */
/* Scores                                                                                    */
/* ---------------------------------------------------------------------------------------- */

/* Sequential float32 score of one (query, row) pair.
 * dot/cosine: tests/cpp/cpu_reference.hpp:12-24 (sum of products in dimension order; cosine is
 * a raw dot product, include/zcgvs/cuda/decode.cuh:30-42);
 * L2: -(sum of squared differences), tests/cpp/test_metrics_filter.cu:16-29. */
static float zo_pair_score(const float* row, const float* query, int dim, int metric) {
    float acc = 0.0f;
    for (int j = 0; j < dim; ++j) {
        if (metric == ZO_L2) {
            const float d = query[j] - row[j];
            acc += d * d;
        } else {
            acc += row[j] * query[j];
        }
    }
    return metric == ZO_L2 ? -acc : acc;
}

/* out[q * n + i] for a float32 (or already-decoded) corpus; mask[i] == 0 gives -FLT_MAX
 * (src/cuda/similarity.cu:109-113). */
void zo_scores_f32(const float* corpus, int64_t n, int dim, const float* queries, int batch,
                   const uint8_t* mask, int metric, float* out) {
    /* Rows are independent; the parallel loop changes no result. */
    for (int q = 0; q < batch; ++q) {
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < n; ++i) {
            float value;
            if (mask != NULL && mask[i] == 0) {
                value = -FLT_MAX;
            } else {
                value = zo_pair_score(corpus + i * dim, queries + (int64_t)q * dim, dim, metric);
            }
            out[(int64_t)q * n + i] = value;
        }
    }
}

/* ---------------------------------------------------------------------------------------- */
/* Storage conversions                                                                       */
/* ---------------------------------------------------------------------------------------- */

/* IEEE binary16 -> binary32, exact. */
static float zo_half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t exponent = (h >> 10) & 0x1Fu;
    const uint32_t mantissa = h & 0x3FFu;
    uint32_t bits;
    if (exponent == 0) {
        if (mantissa == 0) {
            bits = sign;
        } else { /* subnormal: value = mantissa * 2^-24 */
            float value = (float)mantissa * 5.9604644775390625e-08f;
            memcpy(&bits, &value, 4);
            bits |= sign;
        }
    } else if (exponent == 31) {
        bits = sign | 0x7F800000u | (mantissa << 13);
    } else {
        bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

/* IEEE binary32 -> binary16, round to nearest even (the __float2half conversion of
 * src/cuda/convert.cu:17-23). */
static uint16_t zo_float_to_half(float value) {
    uint32_t bits;
    memcpy(&bits, &value, 4);
    const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    const uint32_t exponent = (bits >> 23) & 0xFFu;
    uint32_t mantissa = bits & 0x7FFFFFu;
    if (exponent == 0xFFu) { /* inf / nan */
        return (uint16_t)(sign | 0x7C00u | (mantissa ? 0x200u | (mantissa >> 13) : 0u));
    }
    const int e = (int)exponent - 127;
    if (e > 15) {
        return (uint16_t)(sign | 0x7C00u); /* overflow -> inf */
    }
    if (e >= -14) { /* normal half */
        uint32_t h = ((uint32_t)(e + 15) << 10) | (mantissa >> 13);
        const uint32_t rest = mantissa & 0x1FFFu;
        if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) {
            h += 1u; /* may carry into the exponent, which is the correct rounding */
        }
        return (uint16_t)(sign | h);
    }
    if (e < -25) {
        return sign; /* rounds to zero */
    }
    /* subnormal half: value = m * 2^-24 with m = round(significand * 2^(e + 1)), where the
     * 24-bit significand includes the implicit bit; e in [-25, -15] drops 14..24 bits. */
    mantissa |= 0x800000u;
    const int total_shift = -e - 1;
    uint32_t h = mantissa >> total_shift;
    const uint32_t rest = mantissa & ((1u << total_shift) - 1u);
    const uint32_t halfway = 1u << (total_shift - 1);
    if (rest > halfway || (rest == halfway && (h & 1u))) {
        h += 1u;
    }
    return (uint16_t)(sign | h);
}

void zo_f32_to_f16(const float* src, int64_t count, uint16_t* dst) {
    for (int64_t i = 0; i < count; ++i) {
        dst[i] = zo_float_to_half(src[i]);
    }
}

void zo_f16_to_f32(const uint16_t* src, int64_t count, float* dst) {
    for (int64_t i = 0; i < count; ++i) {
        dst[i] = zo_half_to_float(src[i]);
    }
}

/* q = clamp(nearbyint(x * (1/scale)), -127, 127), the reciprocal rule of
 * src/cuda/convert.cu:25-32 and tests/cpp/cpu_reference.hpp:51-62 (scale <= 0 -> reciprocal 0). */
void zo_quantize_i8(const float* src, int64_t count, float scale, int8_t* dst) {
    const float inverse = scale > 0.0f ? 1.0f / scale : 0.0f;
    for (int64_t i = 0; i < count; ++i) {
        float q = nearbyintf(src[i] * inverse);
        q = fminf(127.0f, fmaxf(-127.0f, q));
        dst[i] = (int8_t)q;
    }
}

/* int8 * scale as float32 (include/zcgvs/cuda/decode.cuh:24-26). */
void zo_dequantize_i8(const int8_t* src, int64_t count, float scale, float* dst) {
    for (int64_t i = 0; i < count; ++i) {
        dst[i] = (float)src[i] * scale;
    }
}

/* tests/cpp/cpu_reference.hpp:51-62: quantize with the reciprocal rule, then dequantize. */
void zo_quantize_dequantize_i8(const float* src, int64_t count, float scale, float* dst) {
    const float inverse = scale > 0.0f ? 1.0f / scale : 0.0f;
    for (int64_t i = 0; i < count; ++i) {
        float q = nearbyintf(src[i] * inverse);
        q = fminf(127.0f, fmaxf(-127.0f, q));
        dst[i] = q * scale;
    }
}

/* Per-row symmetric int8 (no reference counterpart; the per-vector configuration): s = max|x|/127
 * (1 for an all-zero row), codes by the reciprocal rule above. */
void zo_quantize_rows_i8(const float* src, int64_t rows, int dim, int8_t* dst, float* scales) {
    for (int64_t r = 0; r < rows; ++r) {
        const float* x = src + r * dim;
        float peak = 0.0f;
        for (int j = 0; j < dim; ++j) {
            peak = fmaxf(peak, fabsf(x[j]));
        }
        const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
        scales[r] = scale;
        zo_quantize_i8(x, dim, scale, dst + r * dim);
    }
}

/* Per-vector int8 x int8 score: exact int32 dot, then (float)dot * (s_q * s_r) in that order. */
void zo_scores_i8i8(const int8_t* corpus, const float* row_scales, int64_t n, int dim,
                    const int8_t* queries, const float* query_scales, int batch,
                    const uint8_t* mask, float* out) {
    for (int q = 0; q < batch; ++q) {
        const int8_t* qv = queries + (int64_t)q * dim;
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < n; ++i) {
            float value;
            if (mask != NULL && mask[i] == 0) {
                value = -FLT_MAX;
            } else {
                const int8_t* row = corpus + i * dim;
                int32_t dot = 0;
                for (int j = 0; j < dim; ++j) {
                    dot += (int32_t)row[j] * (int32_t)qv[j];
                }
                const float combined = query_scales[q] * row_scales[i];
                value = (float)dot * combined;
            }
            out[(int64_t)q * n + i] = value;
        }
    }
}

/* Sign bits: bit b of word w is dimension 32w + b, set iff x >= 0; padding bits stay 0
 * (tests/cpp/cpu_reference.hpp:64-78, src/cuda/convert.cu:34-53). */
void zo_pack_binary(const float* src, int64_t rows, int dim, uint32_t* dst) {
    const int words = (dim + 31) / 32;
    memset(dst, 0, (size_t)(rows * words) * sizeof(uint32_t));
    for (int64_t r = 0; r < rows; ++r) {
        for (int j = 0; j < dim; ++j) {
            if (src[r * dim + j] >= 0.0f) {
                dst[r * words + j / 32] |= 1u << (j % 32);
            }
        }
    }
}

/* Kernighan popcount of the XOR (tests/cpp/cpu_reference.hpp:80-90). */
int zo_hamming(const uint32_t* a, const uint32_t* b, int words) {
    int distance = 0;
    for (int w = 0; w < words; ++w) {
        uint32_t x = a[w] ^ b[w];
        while (x != 0u) {
            x &= x - 1u;
            ++distance;
        }
    }
    return distance;
}

/* (dim - 2h) / dim in float32 (include/zcgvs/cuda/decode.cuh:45-47); mask -> -FLT_MAX. */
void zo_scores_hamming(const uint32_t* corpus, int64_t n, int dim, const uint32_t* queries,
                       int batch, const uint8_t* mask, float* out) {
    const int words = (dim + 31) / 32;
    for (int q = 0; q < batch; ++q) {
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < n; ++i) {
            float value;
            if (mask != NULL && mask[i] == 0) {
                value = -FLT_MAX;
            } else {
                const int h = zo_hamming(corpus + i * words, queries + (int64_t)q * words, words);
                value = (float)(dim - 2 * h) / (float)dim;
            }
            out[(int64_t)q * n + i] = value;
        }
    }
}

/* L2-normalize rows in place: float32 sum of squares in dimension order, sqrt, divide
 * (tests/cpp/cpu_reference.hpp:36-49). */
void zo_l2_normalize(float* values, int64_t rows, int dim) {
    for (int64_t r = 0; r < rows; ++r) {
        float* x = values + r * dim;
        float norm = 0.0f;
        for (int j = 0; j < dim; ++j) {
            norm += x[j] * x[j];
        }
        norm = sqrtf(norm);
        if (norm <= 0.0f) {
            continue;
        }
        for (int j = 0; j < dim; ++j) {
            x[j] /= norm;
        }
    }
}

/* ---------------------------------------------------------------------------------------- */
/* Selection                                                                                 */
/* ---------------------------------------------------------------------------------------- */

/* 1 if (sa, ia) ranks before (sb, ib). */
static int zo_better(float sa, int64_t ia, float sb, int64_t ib) {
    const int na = isnan(sa);
    const int nb = isnan(sb);
    if (na || nb) {
        if (na && nb) {
            return ia < ib;
        }
        return nb; /* a number beats NaN */
    }
    if (sa > sb) {
        return 1;
    }
    if (sa < sb) {
        return 0;
    }
    return ia < ib;
}

typedef struct {
    float score;
    int64_t index;
} zo_hit;

/* Min-heap on rank: heap[0] is the worst of the kept hits. */
static void zo_sift_down(zo_hit* heap, int size, int i) {
    for (;;) {
        int worst = i;
        const int l = 2 * i + 1;
        const int r = l + 1;
        if (l < size && zo_better(heap[worst].score, heap[worst].index, heap[l].score, heap[l].index)) {
            worst = l;
        }
        if (r < size && zo_better(heap[worst].score, heap[worst].index, heap[r].score, heap[r].index)) {
            worst = r;
        }
        if (worst == i) {
            return;
        }
        const zo_hit t = heap[i];
        heap[i] = heap[worst];
        heap[worst] = t;
        i = worst;
    }
}

static void zo_sift_up(zo_hit* heap, int i) {
    while (i > 0) {
        const int parent = (i - 1) / 2;
        if (zo_better(heap[i].score, heap[i].index, heap[parent].score, heap[parent].index)) {
            return; /* child is better than parent: min-heap order holds */
        }
        const zo_hit t = heap[i];
        heap[i] = heap[parent];
        heap[parent] = t;
        i = parent;
    }
}

static int zo_hit_compare(const void* a, const void* b) {
    const zo_hit* x = (const zo_hit*)a;
    const zo_hit* y = (const zo_hit*)b;
    if (zo_better(x->score, x->index, y->score, y->index)) {
        return -1;
    }
    if (zo_better(y->score, y->index, x->score, x->index)) {
        return 1;
    }
    return 0;
}

/* The k best (score, index) of each [batch, n] row, in rank order; the same result as
 * std::stable_sort by descending score over ascending indices, truncated to k
 * (tests/cpp/cpu_reference.hpp:26-34). Slots past n are (-1, -FLT_MAX) (src/cuda/topk.cu:49-50). */
void zo_topk(const float* scores, int64_t n, int batch, int k, int32_t* out_index,
             float* out_score) {
    /* Queries are independent; the parallel loop changes no result. */
#pragma omp parallel for schedule(dynamic, 1)
    for (int q = 0; q < batch; ++q) {
        zo_hit* heap = (zo_hit*)malloc(sizeof(zo_hit) * (size_t)(k > 0 ? k : 1));
        const float* row = scores + (int64_t)q * n;
        int size = 0;
        for (int64_t i = 0; i < n; ++i) {
            if (size < k) {
                heap[size].score = row[i];
                heap[size].index = i;
                zo_sift_up(heap, size);
                ++size;
            } else if (k > 0 && zo_better(row[i], i, heap[0].score, heap[0].index)) {
                heap[0].score = row[i];
                heap[0].index = i;
                zo_sift_down(heap, size, 0);
            }
        }
        qsort(heap, (size_t)size, sizeof(zo_hit), zo_hit_compare);
        for (int i = 0; i < k; ++i) {
            out_index[(int64_t)q * k + i] = i < size ? (int32_t)heap[i].index : -1;
            out_score[(int64_t)q * k + i] = i < size ? heap[i].score : -FLT_MAX;
        }
        free(heap);
    }
}

/* ---------------------------------------------------------------------------------------- */
/* Rescore and lexical stages                                                               */
/* ---------------------------------------------------------------------------------------- */

/* Exact score of each candidate row (decoded float32 store) against its float32 query; an
 * index < 0 or >= n gives -FLT_MAX (src/cuda/rescore.cu:33-63). */
void zo_rescore(const float* store, int64_t n, int dim, const float* queries, int batch,
                const int32_t* candidates, int count, int metric, float* out) {
    for (int q = 0; q < batch; ++q) {
        for (int s = 0; s < count; ++s) {
            const int32_t doc = candidates[(int64_t)q * count + s];
            float value = -FLT_MAX;
            if (doc >= 0 && doc < n) {
                value = zo_pair_score(store + (int64_t)doc * dim, queries + (int64_t)q * dim, dim, metric);
            }
            out[(int64_t)q * count + s] = value;
        }
    }
}

/* out[i] = candidates[local[i]] for local in [0, count), else -1 (src/cuda/rescore.cu:65-79). */
void zo_remap(const int32_t* candidates, const int32_t* local, int count, int k, int batch,
              int32_t* out) {
    for (int q = 0; q < batch; ++q) {
        for (int i = 0; i < k; ++i) {
            const int32_t l = local[(int64_t)q * k + i];
            out[(int64_t)q * k + i] = (l >= 0 && l < count) ? candidates[(int64_t)q * count + l] : -1;
        }
    }
}

/* BM25 accumulation of one query: for each term slot in order (terms < 0 skipped), add every
 * posting weight to its document (documents outside [0, n) skipped); tests/cpp/test_lexical.cu:
 * 71-80 and src/cuda/lexical.cu:17-42. `out` is zeroed here. */
void zo_bm25(const int64_t* offsets, const int32_t* docs, const float* weights,
             const int32_t* terms, int term_count, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) {
        out[i] = 0.0f;
    }
    for (int t = 0; t < term_count; ++t) {
        const int32_t term = terms[t];
        if (term < 0) {
            continue;
        }
        for (int64_t p = offsets[term]; p < offsets[term + 1]; ++p) {
            const int32_t doc = docs[p];
            if (doc >= 0 && doc < n) {
                out[doc] += weights[p];
            }
        }
    }
}

/* max(0, max_i values[i]) (src/cuda/lexical.cu:44-65). */
float zo_max_positive(const float* values, int64_t n) {
    float best = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        best = fmaxf(best, values[i]);
    }
    return best;
}

/* dense[i] = w * dense[i] + (1 - w) * lexical[i] * inverse, inverse = max > 0 ? 1/max : 0
 * (src/cuda/lexical.cu:67-74), each operation rounded separately. */
void zo_fuse(float* dense, const float* lexical, float lexical_max, float weight, int64_t n) {
    const float inverse = lexical_max > 0.0f ? 1.0f / lexical_max : 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        dense[i] = weight * dense[i] + (1.0f - weight) * lexical[i] * inverse;
    }
}

/* BM25 posting weight of python/zcgvs_tools/build_lexical.py:143-154, evaluated in double:
 * idf = ln(1 + (N - df + 0.5) / (df + 0.5)),
 * w = idf * tf * (k1 + 1) / (tf + k1 * (1 - b + b * len / avgdl)), then rounded to float32. */
float zo_bm25_weight(int64_t doc_count, int64_t df, int32_t tf, double length,
                     double average_length, double k1, double b) {
    const double normalizer = k1 * (1.0 - b + b * length / average_length);
    const double idf = log(1.0 + ((double)doc_count - (double)df + 0.5) / ((double)df + 0.5));
    const double weight = idf * ((double)tf * (k1 + 1.0)) / ((double)tf + normalizer);
    return (float)weight;
}

/* Threads the OpenMP loops above use (1 when built without OpenMP). */
#ifdef _OPENMP
#include <omp.h>
#endif
int zo_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* Sets the thread count of the OpenMP loops (results do not depend on it). */
void zo_set_threads(int threads) {
#ifdef _OPENMP
    omp_set_num_threads(threads > 0 ? threads : 1);
#else
    (void)threads;
#endif
}
