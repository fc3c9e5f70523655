"""The single-pass scan of the fused search (single_pass.hip) against the oracle.

A search of at most four queries that no MFMA scan takes is one streaming launch plus one merge
(two for wide selections: groups of workgroup lists first): every workgroup keeps its exact
top-width per query (k, or the rescore candidates C, up to 1024) in LDS and the merges select the
global top-width from those lists.
Each case checks that this path ran (one phase over the whole corpus) and that the result is the
oracle's top-k: bit for bit for the integer kinds (Hamming, per-vector int8) and for exactly
representable scores, to the float32 summation tolerance otherwise. The corpora include the
ones that stress the per-workgroup lists: ascending scores (every row beats the running
threshold, so the lists compact at every check), all-equal scores (lowest indices across
workgroup boundaries), fewer rows than workgroups, masks that leave fewer live rows than k, and
selections of 100 to 1024 keys, which compact their lists repeatedly and merge in groups."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from helpers import assert_topk_equivalent, float_tolerance, normalized
from zcgvs_tools import lexical

pytestmark = pytest.mark.gpu


def _single(capi, desc, n):
    assert capi.search_phase_rows(desc) == [n], "expected the single-pass scan"
    idx, val, flags = capi.search(desc)
    assert not flags.any()
    return idx, val


@pytest.mark.parametrize("batch,metric,dim,k,masked", [
    (1, oracle.COSINE, 384, 10, False),
    (2, oracle.L2, 128, 32, True),
    (3, oracle.DOT, 768, 1, False),
    (4, oracle.COSINE, 1024, 17, True),
])
def test_float32(gpu, batch, metric, dim, k, masked):
    capi = gpu
    n = 200_003
    corpus, queries = normalized(n, dim, 101), normalized(batch, dim, 102)
    mask = (np.random.default_rng(103).random(n) > 0.4).astype(np.uint8) if masked else None
    desc = capi.search_desc(capi.store_desc(capi.DeviceArray.from_host(corpus), n, dim, capi.F32),
                            capi.DeviceArray.from_host(queries), batch, k, metric,
                            mask=capi.DeviceArray.from_host(mask) if masked else None)
    idx, val = _single(capi, desc, n)
    ref = oracle.scores_f32(corpus, queries, metric, mask)
    assert_topk_equivalent(idx, val, ref, k, float_tolerance(queries, corpus, metric))


@pytest.mark.parametrize("n", [5183, 1_000_000])
def test_float16(gpu, n):
    capi = gpu
    dim, batch, k = 384, 1, 10
    half = oracle.f32_to_f16(normalized(n, dim, 111))
    queries = normalized(batch, dim, 112)
    desc = capi.search_desc(capi.store_desc(capi.DeviceArray.from_host(half), n, dim, capi.F16),
                            capi.DeviceArray.from_host(queries), batch, k)
    idx, val = _single(capi, desc, n)
    decoded = half.astype(np.float32)
    assert_topk_equivalent(idx, val, oracle.scores_f32(decoded, queries), k, float_tolerance(queries, decoded, 0))


def test_int8_matrix_scale(gpu):
    capi = gpu
    n, dim, batch, k = 150_000, 256, 2, 20
    corpus, queries = normalized(n, dim, 121), normalized(batch, dim, 122)
    scale = float(np.abs(corpus).max() / 127.0)
    codes = oracle.quantize_i8(corpus, scale)
    desc = capi.search_desc(capi.store_desc(capi.DeviceArray.from_host(codes), n, dim, capi.I8, scale),
                            capi.DeviceArray.from_host(queries), batch, k)
    idx, val = _single(capi, desc, n)
    decoded = oracle.dequantize_i8(codes, scale)
    assert_topk_equivalent(idx, val, oracle.scores_f32(decoded, queries), k, float_tolerance(queries, decoded, 0))


@pytest.mark.parametrize("batch,masked", [(1, False), (4, True)])
def test_int8_per_vector_bit_exact(gpu, batch, masked):
    capi = gpu
    n, dim, k = 300_000, 768, 32
    codes, scales = oracle.quantize_rows_i8(normalized(n, dim, 131))
    queries = normalized(batch, dim, 132)
    mask = (np.random.default_rng(133).random(n) > 0.2).astype(np.uint8) if masked else None
    desc = capi.search_desc(capi.store_desc(capi.DeviceArray.from_host(codes), n, dim, capi.I8, 1.0,
                                            capi.DeviceArray.from_host(scales)),
                            capi.DeviceArray.from_host(queries), batch, k, int8_mode=capi.INT8_PER_VECTOR,
                            mask=capi.DeviceArray.from_host(mask) if masked else None)
    idx, val = _single(capi, desc, n)
    qcodes, qscales = oracle.quantize_rows_i8(queries)
    assert_topk_equivalent(idx, val, oracle.scores_i8i8(codes, scales, qcodes, qscales, mask), k)


@pytest.mark.parametrize("dim", [256, 1024])
def test_binary_bit_exact_with_ties(gpu, dim):
    """Rows drawn from 48 distinct sign patterns: every Hamming score is shared by thousands of
    rows spread over every workgroup, so each top-k ends inside a tie (lowest indices first)."""
    capi = gpu
    n, batch, k = 250_000, 3, 32
    base = normalized(48, dim, 141)
    rows = base[np.random.default_rng(142).integers(0, 48, n)]
    words = oracle.pack_binary(rows)
    queries = normalized(batch, dim, 143)
    desc = capi.search_desc(capi.store_desc(capi.DeviceArray.from_host(words), n, dim, capi.BINARY),
                            capi.DeviceArray.from_host(queries), batch, k)
    idx, val = _single(capi, desc, n)
    assert_topk_equivalent(idx, val, oracle.scores_hamming(words, oracle.pack_binary(queries), dim), k)


def test_binary_with_float16_rescore(gpu):
    capi = gpu
    n, dim, batch, k, c = 120_000, 512, 2, 10, 32
    rows = normalized(n, dim, 151)
    words, half = oracle.pack_binary(rows), oracle.f32_to_f16(rows)
    queries = normalized(batch, dim, 152)
    d_words, d_q = capi.DeviceArray.from_host(words), capi.DeviceArray.from_host(queries)
    stage1 = capi.search_desc(capi.store_desc(d_words, n, dim, capi.BINARY), d_q, batch, c)
    cand, cand_val = _single(capi, stage1, n)
    assert_topk_equivalent(cand, cand_val, oracle.scores_hamming(words, oracle.pack_binary(queries), dim), c)
    full = capi.search_desc(capi.store_desc(d_words, n, dim, capi.BINARY), d_q, batch, k,
                            rescore=capi.store_desc(capi.DeviceArray.from_host(half), n, dim, capi.F16),
                            rescore_candidates=c)
    idx, val = _single(capi, full, n)
    decoded = half.astype(np.float32)
    for b in range(batch):
        rescored = oracle.rescore(decoded, queries[b:b + 1], cand[b:b + 1])
        local, ref_val = oracle.topk(rescored, k)
        tol = float_tolerance(queries[b:b + 1], decoded[cand[b]], 0)
        for r in range(k):
            g, e = int(idx[b, r]), int(cand[b, local[0, r]])
            assert g in set(cand[b].tolist())
            if g != e:
                pos = int(np.flatnonzero(cand[b] == g)[0])
                assert abs(float(rescored[0, pos]) - float(ref_val[0, r])) <= tol[0, pos] + tol[0, local[0, r]]


def test_hybrid(gpu):
    capi = gpu
    n, vocab, dim, batch, k, w = 60_000, 5000, 384, 2, 10, 0.6
    index = lexical.synthetic_index(n, vocab, seed=161)
    terms = lexical.synthetic_queries(batch, 8, vocab, seed=162)
    half = oracle.f32_to_f16(normalized(n, dim, 163))
    queries = normalized(batch, dim, 164)
    desc = capi.search_desc(capi.store_desc(capi.DeviceArray.from_host(half), n, dim, capi.F16),
                            capi.DeviceArray.from_host(queries), batch, k,
                            lex_offsets=capi.DeviceArray.from_host(index["offsets"]),
                            lex_docs=capi.DeviceArray.from_host(index["posting_docs"]),
                            lex_weights=capi.DeviceArray.from_host(index["posting_weights"]), lex_doc_count=n,
                            lex_vocab_size=vocab, query_terms=capi.DeviceArray.from_host(terms), lexical_stride=8,
                            dense_weight=w, flags=capi.SEARCH_SORTED_POSTINGS)
    idx, val = _single(capi, desc, n)
    decoded = half.astype(np.float32)
    dense = oracle.scores_f32(decoded, queries)
    fused = np.empty_like(dense)
    for b in range(batch):
        lex = oracle.bm25(index["offsets"], index["posting_docs"], index["posting_weights"], terms[b], n)
        fused[b] = oracle.fuse(dense[b], lex, oracle.max_positive(lex), w)
    tol = np.float32(w) * float_tolerance(queries, decoded, 0) + 1e-6
    assert_topk_equivalent(idx, val, fused, k, tol)


def _ramp(n, dim, ascending):
    """Rows whose dot product with e0 is exactly float32(i) (ascending) or float32(n - i): every
    score is exact, so the result is checked bit for bit."""
    corpus = np.zeros((n, dim), np.float32)
    corpus[:, 0] = np.arange(n, dtype=np.float32) if ascending else np.arange(n, 0, -1, dtype=np.float32)
    query = np.zeros((1, dim), np.float32)
    query[0, 0] = 1.0
    return corpus, query


@pytest.mark.parametrize("ascending", [True, False])
@pytest.mark.parametrize("k", [1, 32, 100])
def test_monotone_scores(gpu, ascending, k):
    capi = gpu
    n, dim = 400_000, 64
    corpus, query = _ramp(n, dim, ascending)
    desc = capi.search_desc(capi.store_desc(capi.DeviceArray.from_host(corpus), n, dim, capi.F32),
                            capi.DeviceArray.from_host(query), 1, k, oracle.DOT)
    idx, val = _single(capi, desc, n)
    assert_topk_equivalent(idx, val, oracle.scores_f32(corpus, query, oracle.DOT), k)
    expected = list(range(n - 1, n - 1 - k, -1)) if ascending else list(range(k))
    assert idx[0].tolist() == expected


@pytest.mark.parametrize("n", [1, 20, 100, 255, 257, 5183])
def test_small_corpora(gpu, n):
    """Fewer rows than workgroups leaves most row ranges empty; k = min(n, 20) takes the whole
    corpus when it is that small."""
    capi = gpu
    dim, batch = 128, 2
    k = min(n, 20)
    corpus, queries = normalized(n, dim, 171), normalized(batch, dim, 172)
    desc = capi.search_desc(capi.store_desc(capi.DeviceArray.from_host(corpus), n, dim, capi.F32),
                            capi.DeviceArray.from_host(queries), batch, k)
    idx, val = _single(capi, desc, n)
    assert_topk_equivalent(idx, val, oracle.scores_f32(corpus, queries), k, float_tolerance(queries, corpus, 0))


@pytest.mark.parametrize("k", [32, 100])
def test_constant_scores_take_the_lowest_indices(gpu, k):
    capi = gpu
    n, dim = 300_000, 64
    corpus = np.zeros((n, dim), np.float32)
    corpus[:, 0] = 1.0
    query = np.zeros((1, dim), np.float32)
    query[0, 0] = 0.5
    desc = capi.search_desc(capi.store_desc(capi.DeviceArray.from_host(corpus), n, dim, capi.F32),
                            capi.DeviceArray.from_host(query), 1, k)
    idx, val = _single(capi, desc, n)
    assert idx[0].tolist() == list(range(k)) and np.all(val == 0.5)


def test_mask_leaves_fewer_rows_than_k(gpu):
    """Five live rows and k = 12: the five by score, then masked rows (score -FLT_MAX) by index."""
    capi = gpu
    n, dim, k = 100_000, 256, 12
    codes, scales = oracle.quantize_rows_i8(normalized(n, dim, 181))
    query = normalized(1, dim, 182)
    mask = np.zeros(n, np.uint8)
    mask[[7, 4096, 50_000, 77_777, 99_999]] = 1
    desc = capi.search_desc(capi.store_desc(capi.DeviceArray.from_host(codes), n, dim, capi.I8, 1.0,
                                            capi.DeviceArray.from_host(scales)),
                            capi.DeviceArray.from_host(query), 1, k, int8_mode=capi.INT8_PER_VECTOR,
                            mask=capi.DeviceArray.from_host(mask))
    idx, val = _single(capi, desc, n)
    qcodes, qscales = oracle.quantize_rows_i8(query)
    assert_topk_equivalent(idx, val, oracle.scores_i8i8(codes, scales, qcodes, qscales, mask), k)
    assert sorted(idx[0, :5].tolist()) == [7, 4096, 50_000, 77_777, 99_999]
    assert idx[0, 5:].tolist() == [0, 1, 2, 3, 4, 5, 6]


def test_integer_kinds_match_the_phased_scan(gpu):
    """The single pass and the phased scan with its exact fallback return the same keys."""
    capi = gpu
    n, dim, batch, k = 200_000, 512, 4, 24
    words = oracle.pack_binary(normalized(n, dim, 191))
    d_words = capi.DeviceArray.from_host(words)
    d_q = capi.DeviceArray.from_host(normalized(batch, dim, 192))
    single = capi.search_desc(capi.store_desc(d_words, n, dim, capi.BINARY), d_q, batch - 1, k)
    phased = capi.search_desc(capi.store_desc(d_words, n, dim, capi.BINARY), d_q, batch - 1, k,
                              flags=capi.SEARCH_FORCE_EXACT_PASS)
    assert len(capi.search_phase_rows(phased)) > 1
    a, av = _single(capi, single, n)
    b, bv, _ = capi.search(phased)
    assert np.array_equal(a, b) and np.array_equal(av, bv)


def test_selection_limits(gpu):
    """Four queries and k = 1024 is the widest single pass; five queries and the test flags take
    the phased scan. (A dimension the MFMA float scan does not take, which would take four
    unmasked queries of 128 to 512 dimensions.)"""
    capi = gpu
    n, dim = 50_000, 64
    d_corpus = capi.DeviceArray.from_host(normalized(n, dim, 201))
    d_q = capi.DeviceArray.from_host(normalized(5, dim, 202))
    store = capi.store_desc(d_corpus, n, dim, capi.F32)
    assert capi.search_phase_rows(capi.search_desc(store, d_q, 4, 32)) == [n]
    assert capi.search_phase_rows(capi.search_desc(store, d_q, 4, 1024)) == [n]
    assert capi.search_phase_rows(capi.search_desc(store, d_q, 5, 10)) != [n]
    for flag in (capi.SEARCH_FORCE_EXACT_PASS, capi.SEARCH_TEST_TINY_SEGMENTS):
        assert capi.search_phase_rows(capi.search_desc(store, d_q, 1, 10, flags=flag)) != [n]


@pytest.mark.parametrize("batch,k,masked", [(1, 100, False), (2, 333, True), (4, 1024, False)])
def test_wide_selections_float32(gpu, batch, k, masked):
    # (96 dimensions: the MFMA float scan, which takes four unmasked queries of 128 to 512
    # dimensions, does not take them)
    capi = gpu
    n, dim = 400_009, 96
    corpus, queries = normalized(n, dim, 211), normalized(batch, dim, 212)
    mask = (np.random.default_rng(213).random(n) > 0.5).astype(np.uint8) if masked else None
    desc = capi.search_desc(capi.store_desc(capi.DeviceArray.from_host(corpus), n, dim, capi.F32),
                            capi.DeviceArray.from_host(queries), batch, k, oracle.L2 if masked else oracle.DOT,
                            mask=capi.DeviceArray.from_host(mask) if masked else None)
    idx, val = _single(capi, desc, n)
    metric = oracle.L2 if masked else oracle.DOT
    ref = oracle.scores_f32(corpus, queries, metric, mask)
    assert_topk_equivalent(idx, val, ref, k, float_tolerance(queries, corpus, metric))


def test_wide_selection_int8_per_vector_bit_exact(gpu):
    capi = gpu
    n, dim, batch, k = 500_000, 768, 1, 100
    codes, scales = oracle.quantize_rows_i8(normalized(n, dim, 221))
    queries = normalized(batch, dim, 222)
    desc = capi.search_desc(capi.store_desc(capi.DeviceArray.from_host(codes), n, dim, capi.I8, 1.0,
                                            capi.DeviceArray.from_host(scales)),
                            capi.DeviceArray.from_host(queries), batch, k, int8_mode=capi.INT8_PER_VECTOR)
    idx, val = _single(capi, desc, n)
    qcodes, qscales = oracle.quantize_rows_i8(queries)
    assert_topk_equivalent(idx, val, oracle.scores_i8i8(codes, scales, qcodes, qscales), k)


def test_wide_binary_with_ties_and_rescore(gpu):
    """Hamming top-1000 over 64 repeated sign patterns (the top-1000 ends inside a tie of
    thousands of rows: lowest indices, bit for bit), then the float16 rescore of those 1000."""
    capi = gpu
    n, dim, batch, k, c = 300_000, 1024, 1, 10, 1000
    base = normalized(64, dim, 231)
    rows = base[np.random.default_rng(232).integers(0, 64, n)] + 1e-3 * normalized(n, dim, 233)
    words, half = oracle.pack_binary(rows), oracle.f32_to_f16(rows)
    queries = normalized(batch, dim, 234)
    d_words, d_q = capi.DeviceArray.from_host(words), capi.DeviceArray.from_host(queries)
    stage1 = capi.search_desc(capi.store_desc(d_words, n, dim, capi.BINARY), d_q, batch, c)
    cand, cand_val = _single(capi, stage1, n)
    assert_topk_equivalent(cand, cand_val, oracle.scores_hamming(words, oracle.pack_binary(queries), dim), c)
    full = capi.search_desc(capi.store_desc(d_words, n, dim, capi.BINARY), d_q, batch, k,
                            rescore=capi.store_desc(capi.DeviceArray.from_host(half), n, dim, capi.F16),
                            rescore_candidates=c)
    idx, val = _single(capi, full, n)
    decoded = half.astype(np.float32)
    rescored = oracle.rescore(decoded, queries, cand)
    local, ref_val = oracle.topk(rescored, k)
    tol = float_tolerance(queries, decoded[cand[0]], 0)
    for r in range(k):
        g, e = int(idx[0, r]), int(cand[0, local[0, r]])
        assert g in set(cand[0].tolist())
        if g != e:
            pos = int(np.flatnonzero(cand[0] == g)[0])
            assert abs(float(rescored[0, pos]) - float(ref_val[0, r])) <= tol[0, pos] + tol[0, local[0, r]]


@pytest.mark.parametrize("ascending", [True, False])
def test_wide_monotone_scores(gpu, ascending):
    """Ascending scores append every row to every list: with k = 1000 each list compacts many
    times and the merges see full groups."""
    capi = gpu
    n, dim, k = 600_000, 64, 1000
    corpus, query = _ramp(n, dim, ascending)
    desc = capi.search_desc(capi.store_desc(capi.DeviceArray.from_host(corpus), n, dim, capi.F32),
                            capi.DeviceArray.from_host(query), 1, k, oracle.DOT)
    idx, val = _single(capi, desc, n)
    expected = list(range(n - 1, n - 1 - k, -1)) if ascending else list(range(k))
    assert idx[0].tolist() == expected
    assert_topk_equivalent(idx, val, oracle.scores_f32(corpus, query, oracle.DOT), k)


def test_wide_selection_small_corpus(gpu):
    """1,500 rows and k = 1,000: most workgroups hold a handful of rows, the groups' merges see
    mostly empty segments."""
    capi = gpu
    n, dim, k = 1_500, 128, 1_000
    corpus, queries = normalized(n, dim, 241), normalized(3, dim, 242)
    desc = capi.search_desc(capi.store_desc(capi.DeviceArray.from_host(corpus), n, dim, capi.F32),
                            capi.DeviceArray.from_host(queries), 3, k)
    idx, val = _single(capi, desc, n)
    assert_topk_equivalent(idx, val, oracle.scores_f32(corpus, queries), k, float_tolerance(queries, corpus, 0))
