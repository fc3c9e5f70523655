"""Pins the CPU oracle before anything is checked against it.

Each check can fail for a plausible mistake in the oracle: the reference's own known answers
(tests/python/test_formats.py), the reference's own CPU path compiled from its source
(oracle/_ref, tests/cpp/cpu_reference.hpp), and independent restatements in numpy whose result
the mathematics fixes (integer matmul, sequential float32 cumulative sums, numpy's IEEE half
conversion, stable argsort, closed forms).
"""

import math

import numpy as np
import pytest

import oracle

RNG = np.random.default_rng(20241201)


def normalized(rows, dim, rng=RNG):
    x = rng.standard_normal((rows, dim)).astype(np.float32)
    return x / np.linalg.norm(x, axis=1, keepdims=True).astype(np.float32)


# ---- known answers of the reference --------------------------------------------------------

def test_pack_binary_known_answer():
    # tests/python/test_formats.py:36-52: dims 0, 33, 129 set at dim 130 -> words [1, 2, 0, 0, 2]
    matrix = np.full((1, 130), -1.0, dtype=np.float32)
    matrix[0, [0, 33, 129]] = 1.0
    packed = oracle.pack_binary(matrix)
    assert packed.tolist() == [[1, 2, 0, 0, 2]]
    assert packed[0, 4] >> 2 == 0  # padding bits stay zero


def test_pack_binary_zero_sign_and_nan():
    # x >= 0 sets the bit: -0.0 sets it, NaN does not (src/cuda/convert.cu:46)
    packed = oracle.pack_binary(np.array([[-0.0, np.nan, 0.0, -1e-30]], dtype=np.float32))
    assert packed.tolist() == [[0b0101]]


# ---- the reference's own CPU path -----------------------------------------------------------

# Loaded by the tests that use it (never at collection), so a run that selects none of them
# does not map the library.
needs_ref = pytest.mark.skipif(not oracle.REF_PATH.exists(), reason="reference CPU path was not built here")


@pytest.fixture(scope="module")
def ref():
    return oracle.ref()


@needs_ref
def test_scores_match_reference_cpu_bitwise(ref):
    import ctypes
    corpus = normalized(512, 384)
    query = normalized(1, 384)
    expected = np.empty(512, dtype=np.float32)
    ref.ref_cosine_similarity(ctypes.c_void_p(corpus.ctypes.data), 512, 384,
                              ctypes.c_void_p(query.ctypes.data), ctypes.c_void_p(expected.ctypes.data))
    got = oracle.scores_f32(corpus, query, oracle.COSINE)[0]
    assert np.array_equal(got.view(np.uint32), expected.view(np.uint32))


@needs_ref
@pytest.mark.parametrize("quantized", [False, True])
def test_topk_matches_reference_stable_sort(ref, quantized):
    import ctypes
    scores = RNG.uniform(-100, 100, size=5000).astype(np.float32)
    if quantized:  # heavy ties: only 41 distinct values
        scores = np.round(scores / 5.0).astype(np.float32)
    k = 100
    expected = np.empty(k, dtype=np.int32)
    ref.ref_topk_indices(ctypes.c_void_p(scores.ctypes.data), scores.size, k,
                         ctypes.c_void_p(expected.ctypes.data))
    idx, val = oracle.topk(scores, k)
    assert idx[0].tolist() == expected.tolist()
    assert np.array_equal(val[0], scores[expected])


@needs_ref
def test_quantize_dequantize_matches_reference(ref):
    import ctypes
    x = RNG.standard_normal(4096).astype(np.float32)
    # include exact half-way points: (n + 0.5) * scale
    scale = np.float32(1.0 / 127.0)
    x[:64] = (np.arange(64, dtype=np.float32) - 32.0 + 0.5) * scale
    expected = np.empty_like(x)
    ref.ref_quantize_dequantize_i8(ctypes.c_void_p(x.ctypes.data), x.size, ctypes.c_float(scale),
                                   ctypes.c_void_p(expected.ctypes.data))
    got = oracle.quantize_dequantize_i8(x, scale)
    assert np.array_equal(got.view(np.uint32), expected.view(np.uint32))


@needs_ref
def test_pack_and_hamming_match_reference(ref):
    import ctypes
    x = RNG.standard_normal((64, 100)).astype(np.float32)
    expected = np.empty((64, 4), dtype=np.uint32)
    ref.ref_pack_binary(ctypes.c_void_p(x.ctypes.data), 64, 100, ctypes.c_void_p(expected.ctypes.data))
    packed = oracle.pack_binary(x)
    assert np.array_equal(packed, expected)
    for i in range(0, 64, 7):
        h_ref = ref.ref_hamming(ctypes.c_void_p(packed[i].ctypes.data),
                                ctypes.c_void_p(packed[(i + 1) % 64].ctypes.data), 4)
        assert oracle.hamming(packed[i], packed[(i + 1) % 64]) == h_ref


@needs_ref
def test_l2_normalize_matches_reference(ref):
    import ctypes
    x = RNG.standard_normal((4, 97)).astype(np.float32)
    got = oracle.l2_normalize(x)
    for r in range(4):
        row = x[r].copy()
        ref.ref_l2_normalize(ctypes.c_void_p(row.ctypes.data), 97)
        assert np.array_equal(got[r].view(np.uint32), row.view(np.uint32))


# ---- independent restatements -------------------------------------------------------------

def _sequential_dot(corpus, query):
    products = (corpus * query[None, :]).astype(np.float32)
    return np.cumsum(products, axis=1, dtype=np.float32)[:, -1]


@pytest.mark.parametrize("metric", [oracle.COSINE, oracle.DOT, oracle.L2])
def test_scores_f32_sequential_order(metric):
    corpus = normalized(300, 97)
    query = normalized(1, 97)[0]
    got = oracle.scores_f32(corpus, query, metric)[0]
    if metric == oracle.L2:
        diff = (query[None, :] - corpus).astype(np.float32)
        expected = -np.cumsum((diff * diff).astype(np.float32), axis=1, dtype=np.float32)[:, -1]
    else:
        expected = _sequential_dot(corpus, query)
    assert np.array_equal(got, expected)


def test_scores_mask_gives_minus_flt_max():
    corpus = normalized(50, 16)
    mask = (np.arange(50) % 2).astype(np.uint8)
    got = oracle.scores_f32(corpus, corpus[:2], oracle.DOT, mask)
    assert np.all(got[:, mask == 0] == -np.finfo(np.float32).max)
    assert np.all(got[:, mask == 1] > -1.1)


def test_f16_conversion_matches_ieee():
    special = np.array([0.0, -0.0, 65504.0, 65520.0, 1e-8, 6.0e-8, 2.0 ** -25, 2.0 ** -24,
                        3 * 2.0 ** -26, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, np.inf, -np.inf],
                       dtype=np.float32)
    values = np.concatenate([special, RNG.standard_normal(20000).astype(np.float32),
                             (RNG.standard_normal(5000) * 1e-5).astype(np.float32)])
    got = oracle.f32_to_f16(values)
    assert np.array_equal(got.view(np.uint16), values.astype(np.float16).view(np.uint16))
    back = oracle.f16_to_f32(got)
    assert np.array_equal(back, got.astype(np.float32))


def test_quantize_rows_matches_numpy():
    x = normalized(64, 768)
    x[3] = 0.0
    codes, scales = oracle.quantize_rows_i8(x)
    peak = np.max(np.abs(x), axis=1)
    expected_scales = np.where(peak > 0, peak / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    assert np.array_equal(scales, expected_scales)
    inverse = (np.float32(1.0) / expected_scales).astype(np.float32)
    expected = np.clip(np.rint((x * inverse[:, None]).astype(np.float32)), -127, 127).astype(np.int8)
    assert np.array_equal(codes, expected)
    assert np.all(np.abs(codes).max(axis=1)[[0, 1, 2]] == 127)


def test_i8i8_scores_match_integer_matmul():
    x = normalized(500, 768)
    q = normalized(9, 768)
    codes, rs = oracle.quantize_rows_i8(x)
    qcodes, qs = oracle.quantize_rows_i8(q)
    got = oracle.scores_i8i8(codes, rs, qcodes, qs)
    dot = qcodes.astype(np.int64) @ codes.astype(np.int64).T
    combined = (qs[:, None] * rs[None, :]).astype(np.float32)
    expected = (dot.astype(np.float32) * combined).astype(np.float32)
    assert np.array_equal(got, expected)


def test_hamming_closed_forms():
    x = RNG.standard_normal((3, 1024)).astype(np.float32)
    packed = oracle.pack_binary(np.concatenate([x, -x]))  # row r+3 is the complement of row r
    for r in range(3):
        assert oracle.hamming(packed[r], packed[r]) == 0
        assert oracle.hamming(packed[r], packed[r + 3]) == 1024
    scores = oracle.scores_hamming(packed, packed[:1], 1024)[0]
    assert scores[0] == 1.0 and scores[3] == -1.0
    h = np.array([oracle.hamming(packed[0], packed[i]) for i in range(6)])
    assert np.array_equal(scores, ((1024 - 2 * h) / np.float32(1024)).astype(np.float32))


@pytest.mark.parametrize("ties", [False, True])
def test_topk_matches_stable_argsort(ties):
    scores = RNG.standard_normal((3, 20000)).astype(np.float32)
    if ties:
        scores = np.round(scores * 4).astype(np.float32)
        scores[0, :100] = -0.0  # -0.0 ties with +0.0
        scores[1, 5:9] = np.nan
    k = 257
    idx, val = oracle.topk(scores, k)
    for b in range(3):
        key = np.where(np.isnan(scores[b]), np.inf, -scores[b])  # NaN last
        order = np.argsort(key, kind="stable")[:k]
        assert idx[b].tolist() == order.tolist()


def test_topk_pads_when_k_exceeds_n():
    idx, val = oracle.topk(np.array([[3.0, 1.0]], dtype=np.float32), 4)
    assert idx.tolist() == [[0, 1, -1, -1]]
    assert val[0, 2] == -np.finfo(np.float32).max


def test_bm25_weight_pinned_by_its_special_cases():
    """python/zcgvs_tools/build_lexical.py:143-154: w = idf * tf (k1 + 1) / (tf + k1 (1 - b +
    b len / avgdl)), idf = ln(1 + (N - df + 0.5) / (df + 0.5)), in float64, cast to float32.
    Each check below is fixed by the mathematics, not by the formula's text: a dropped term, a
    swapped operand or a wrong constant fails one of them."""
    n, avg = 1_000_000, 201.5
    w = oracle.bm25_weight
    # a term absent from the document contributes nothing
    assert w(n, 10, 0, 150, avg) == 0.0
    # idf alone, from the three closed forms below (k1 = 0 removes the saturation factor)
    for df in (1, 17, 5000, n // 2, n):
        idf = math.log1p((n - df + 0.5) / (df + 0.5))
        for tf in (1, 2, 4, 64):
            assert w(n, df, tf, 123, avg, k1=0.0) == np.float32(idf)
    # a term in every document keeps only the +0.5 smoothing: idf = ln(1 + 0.5 / (N + 0.5))
    assert w(n, n, 1, 100, avg, k1=0.0) == np.float32(math.log1p(0.5 / (n + 0.5)))
    # one document holding the term out of two: idf = ln(1 + 1.5 / 1.5) = ln 2
    assert w(2, 1, 1, 5, 5, k1=0.0) == np.float32(math.log(2.0))
    # b = 0 makes the weight independent of the document length
    base = w(n, 300, 3, 10, avg, b=0.0)
    assert all(w(n, 300, 3, length, avg, b=0.0) == base for length in (1, 200, 5000))
    # at length == avgdl the length factor is 1 for every b: tf (k1 + 1) / (tf + k1)
    idf = math.log1p((n - 300 + 0.5) / (300 + 0.5))
    for b in (0.0, 0.3, 0.75, 1.0):
        assert w(n, 300, 2, avg, avg, b=b) == np.float32(idf * 2 * 2.2 / (2 + 1.2))
    # strictly increasing in tf, bounded by (and tending to) idf * (k1 + 1)
    series = [w(n, 300, tf, 180, avg) for tf in (1, 2, 3, 5, 10, 100, 10_000, 10**8)]
    assert all(a < b for a, b in zip(series, series[1:-1]))
    assert series[-1] <= np.float32(idf * 2.2) and abs(series[-1] - idf * 2.2) < 1e-6 * idf
    # longer documents weigh less (b > 0), rarer terms weigh more
    assert w(n, 300, 3, 100, avg) > w(n, 300, 3, 400, avg)
    assert w(n, 30, 3, 100, avg) > w(n, 300, 3, 100, avg) > w(n, 3000, 3, 100, avg)
    # doubling the length and avgdl together changes nothing
    assert w(n, 300, 3, 150, avg) == w(n, 300, 3, 300, 2 * avg)


def test_bm25_accumulates_in_term_order():
    offsets = np.array([0, 3, 5, 5, 8], dtype=np.int64)
    docs = np.array([0, 2, 9, 2, 3, 0, 2, 7], dtype=np.int32)
    weights = np.array([0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8], dtype=np.float32)
    got = oracle.bm25(offsets, docs, weights, np.array([3, 0, -1, 1], dtype=np.int32), 8)
    expected = np.zeros(8, dtype=np.float32)
    for term in (3, 0, 1):
        for p in range(offsets[term], offsets[term + 1]):
            if docs[p] < 8:
                expected[docs[p]] = np.float32(expected[docs[p]] + weights[p])
    assert np.array_equal(got, expected)
    assert got[2] == np.float32(np.float32(np.float32(0.7) + np.float32(0.2)) + np.float32(0.4))


def test_fuse_special_cases_and_bounds():
    """zo_fuse (src/cuda/lexical.cu:67-74: w * dense + (1 - w) * lex * inv, inv = 1 / max when
    max > 0, else 0) pinned by what the formula forces rather than by restating it:
    w = 1 leaves the dense scores; w = 0 leaves lex * fl(1 / max), so the top lexical document
    scores within an ulp of 1; max = 0 drops the lexical term; for any w in [0, 1] the result
    is a convex combination of dense and lex / max (within rounding) and rises with lex."""
    n = 4000
    dense = RNG.uniform(-1, 1, n).astype(np.float32)
    lexical = RNG.uniform(0, 7, n).astype(np.float32)
    lexical[17] = np.float32(0.0)
    peak = oracle.max_positive(lexical)
    assert peak == lexical.max()
    top = int(np.argmax(lexical))
    inverse = np.float32(1.0) / np.float32(peak)
    # w = 1: the dense score itself (zero lexical weight)
    assert np.array_equal(oracle.fuse(dense, lexical, peak, 1.0), dense)
    # w = 0: the normalized lexical score, one rounding of lex * inverse
    only_lexical = oracle.fuse(dense, lexical, peak, 0.0)
    assert np.array_equal(only_lexical, (lexical * inverse).astype(np.float32))
    assert abs(float(only_lexical[top]) - 1.0) <= float(np.spacing(np.float32(1.0)))
    assert only_lexical[17] == 0.0 and float(only_lexical.min()) >= 0.0
    # max = 0 (no positive lexical score): the lexical term vanishes
    for w in (0.0, 0.25, 0.6):
        assert np.array_equal(oracle.fuse(dense, lexical, 0.0, w), (np.float32(w) * dense).astype(np.float32))
    # convexity: between dense and lex / max, within a few roundings of the operands' size
    normalized_lex = lexical.astype(np.float64) / float(peak)
    for w in RNG.uniform(0, 1, 12):
        got = oracle.fuse(dense, lexical, peak, float(w)).astype(np.float64)
        lo = np.minimum(dense, normalized_lex)
        hi = np.maximum(dense, normalized_lex)
        slack = 4 * np.spacing(np.maximum(np.abs(lo), np.abs(hi)).astype(np.float32)).astype(np.float64)
        assert np.all(got >= lo - slack) and np.all(got <= hi + slack)
        # monotone in lex at fixed dense: sort by lex with one dense value
        same = np.full(n, dense[0], dtype=np.float32)
        order = np.argsort(lexical, kind="stable")
        ranked = oracle.fuse(same, lexical[order], peak, float(w))
        assert np.all(np.diff(ranked.astype(np.float64)) >= 0)
    # the weight is the dense share: w = 0.75 leans three to one towards dense
    w = 0.75
    mixed = oracle.fuse(dense, lexical, peak, w).astype(np.float64)
    expected = w * dense.astype(np.float64) + (1 - w) * normalized_lex
    assert np.all(np.abs(mixed - expected) <= 1e-6)


def test_rescore_and_remap():
    store = normalized(100, 64)
    queries = normalized(2, 64)
    cand = np.array([[5, -1, 99, 100], [0, 1, 2, 3]], dtype=np.int32)
    got = oracle.rescore(store, queries, cand)
    assert got[0, 1] == -np.finfo(np.float32).max and got[0, 3] == -np.finfo(np.float32).max
    assert got[0, 0] == oracle.scores_f32(store[5:6], queries[0])[0, 0]
    local = np.array([[2, 0], [3, 7]], dtype=np.int32)
    assert oracle.remap(cand, local).tolist() == [[99, 5], [3, -1]]
