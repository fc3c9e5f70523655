"""The exact device fallback of the fused search (recover.hip) against the oracle.

ZCGVS_SEARCH_FORCE_EXACT_PASS runs it for every query; ZCGVS_SEARCH_TEST_TINY_SEGMENTS shrinks the
candidate segments to two slots so nearly every query overflows and reaches it through its
overflow flag. Either way the result must be the oracle's top-k (integer kinds bit for bit, float
kinds to the float tolerance), for every storage kind and scan kernel the fused search uses, with
masks, L2, hybrid fusion, rescore, and heavy score ties (lowest index first)."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from helpers import assert_topk_equivalent, float_tolerance, normalized
from zcgvs_tools import lexical

pytestmark = pytest.mark.gpu

MODES = ["force", "tiny"]


def _flags(capi, mode):
    return capi.SEARCH_FORCE_EXACT_PASS if mode == "force" else capi.SEARCH_TEST_TINY_SEGMENTS


def _run(capi, desc, mode, expect_overflow=False):
    idx, val, flags = capi.search(desc)
    if mode == "tiny" and expect_overflow:
        assert flags.any(), "two-slot segments should overflow"
    return idx, val


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("batch,metric,masked", [(1, 0, False), (3, 2, True), (8, 1, False)])
def test_float32(gpu, mode, batch, metric, masked):
    capi = gpu
    n, dim, k = 150_000, 128, 25
    corpus, queries = normalized(n, dim, 31), normalized(batch, dim, 32)
    mask = (np.random.default_rng(33).random(n) > 0.3).astype(np.uint8) if masked else None
    d_corpus, d_q = capi.DeviceArray.from_host(corpus), capi.DeviceArray.from_host(queries)
    d_mask = capi.DeviceArray.from_host(mask) if masked else None
    desc = capi.search_desc(capi.store_desc(d_corpus, n, dim, capi.F32), d_q, batch, k, metric, mask=d_mask,
                            flags=_flags(capi, mode))
    idx, val = _run(capi, desc, mode)
    ref = oracle.scores_f32(corpus, queries, metric, mask)
    assert_topk_equivalent(idx, val, ref, k, float_tolerance(queries, corpus, metric))


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("batch", [1, 16])
def test_float16(gpu, mode, batch):
    capi = gpu
    n, dim, k = 120_000, 384, 10
    half = oracle.f32_to_f16(normalized(n, dim, 41))
    queries = normalized(batch, dim, 42)
    desc = capi.search_desc(capi.store_desc(capi.DeviceArray.from_host(half), n, dim, capi.F16),
                            capi.DeviceArray.from_host(queries), batch, k, flags=_flags(capi, mode))
    idx, val = _run(capi, desc, mode)
    decoded = half.astype(np.float32)
    assert_topk_equivalent(idx, val, oracle.scores_f32(decoded, queries), k, float_tolerance(queries, decoded, 0))


@pytest.mark.parametrize("mode", MODES)
def test_int8_matrix_scale(gpu, mode):
    capi = gpu
    n, dim, batch, k = 90_000, 256, 5, 40
    corpus, queries = normalized(n, dim, 51), normalized(batch, dim, 52)
    scale = float(np.abs(corpus).max() / 127.0)
    codes = oracle.quantize_i8(corpus, scale)
    desc = capi.search_desc(capi.store_desc(capi.DeviceArray.from_host(codes), n, dim, capi.I8, scale),
                            capi.DeviceArray.from_host(queries), batch, k, flags=_flags(capi, mode))
    idx, val = _run(capi, desc, mode)
    decoded = oracle.dequantize_i8(codes, scale)
    assert_topk_equivalent(idx, val, oracle.scores_f32(decoded, queries), k, float_tolerance(queries, decoded, 0))


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("batch", [2, 24])
def test_int8_per_vector_bit_exact(gpu, mode, batch):
    capi = gpu
    n, dim, k = 100_000, 768, 100
    codes, scales = oracle.quantize_rows_i8(normalized(n, dim, 61))
    queries = normalized(batch, dim, 62)
    mask = (np.random.default_rng(63).random(n) > 0.1).astype(np.uint8)
    desc = capi.search_desc(capi.store_desc(capi.DeviceArray.from_host(codes), n, dim, capi.I8, 1.0,
                                            capi.DeviceArray.from_host(scales)),
                            capi.DeviceArray.from_host(queries), batch, k, int8_mode=capi.INT8_PER_VECTOR,
                            mask=capi.DeviceArray.from_host(mask), flags=_flags(capi, mode))
    idx, val = _run(capi, desc, mode, expect_overflow=True)  # ~800 candidates per query and phase
    qcodes, qscales = oracle.quantize_rows_i8(queries)
    assert_topk_equivalent(idx, val, oracle.scores_i8i8(codes, scales, qcodes, qscales, mask), k)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("batch", [1, 6])
def test_binary_with_rescore_and_ties(gpu, mode, batch):
    """Hamming scores of 1024-bit rows built from 64 distinct rows repeated: every score is
    shared by thousands of rows, so the fallback's top-300 ends inside a tie and must take the
    lowest indices (checked bit for bit); the float16 rescore of those candidates follows."""
    capi = gpu
    n, dim, k, c = 80_000, 1024, 10, 300
    base = normalized(64, dim, 71)
    rows = base[np.random.default_rng(72).integers(0, 64, n)]
    rows = rows + 1e-3 * normalized(n, dim, 73)  # rescore scores differ; signs (mostly) do not
    words = oracle.pack_binary(rows)
    half = oracle.f32_to_f16(rows)
    queries = normalized(batch, dim, 74)
    d_words, d_half = capi.DeviceArray.from_host(words), capi.DeviceArray.from_host(half)
    d_q = capi.DeviceArray.from_host(queries)
    stage1 = capi.search_desc(capi.store_desc(d_words, n, dim, capi.BINARY), d_q, batch, c,
                              flags=_flags(capi, mode))
    cand, cand_val = _run(capi, stage1, mode, expect_overflow=True)
    ref_scores = oracle.scores_hamming(words, oracle.pack_binary(queries), dim)
    assert_topk_equivalent(cand, cand_val, ref_scores, c)
    full = capi.search_desc(capi.store_desc(d_words, n, dim, capi.BINARY), d_q, batch, k,
                            rescore=capi.store_desc(d_half, n, dim, capi.F16), rescore_candidates=c,
                            flags=_flags(capi, mode))
    idx, val = _run(capi, full, mode)
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


@pytest.mark.parametrize("mode", MODES)
def test_hybrid(gpu, mode):
    capi = gpu
    n, vocab, dim, batch, k, w = 50_000, 5000, 256, 4, 10, 0.5
    index = lexical.synthetic_index(n, vocab, seed=81)
    terms = lexical.synthetic_queries(batch, 8, vocab, seed=82)
    half = oracle.f32_to_f16(normalized(n, dim, 83))
    queries = normalized(batch, dim, 84)
    desc = capi.search_desc(capi.store_desc(capi.DeviceArray.from_host(half), n, dim, capi.F16),
                            capi.DeviceArray.from_host(queries), batch, k,
                            lex_offsets=capi.DeviceArray.from_host(index["offsets"]),
                            lex_docs=capi.DeviceArray.from_host(index["posting_docs"]),
                            lex_weights=capi.DeviceArray.from_host(index["posting_weights"]), lex_doc_count=n,
                            lex_vocab_size=vocab, query_terms=capi.DeviceArray.from_host(terms), lexical_stride=8,
                            dense_weight=w, flags=_flags(capi, mode) | capi.SEARCH_SORTED_POSTINGS)
    idx, val = _run(capi, desc, mode)
    decoded = half.astype(np.float32)
    dense = oracle.scores_f32(decoded, queries)
    fused = np.empty_like(dense)
    for b in range(batch):
        lex = oracle.bm25(index["offsets"], index["posting_docs"], index["posting_weights"], terms[b], n)
        fused[b] = oracle.fuse(dense[b], lex, oracle.max_positive(lex), w)
    tol = np.float32(w) * float_tolerance(queries, decoded, 0) + 1e-6
    assert_topk_equivalent(idx, val, fused, k, tol)


def test_constant_scores_take_the_lowest_indices(gpu):
    # every row scores exactly the same: the top-k are rows 0..k-1, in order
    capi = gpu
    n, dim, k = 70_000, 64, 50
    corpus = np.zeros((n, dim), np.float32)
    corpus[:, 0] = 1.0
    query = np.zeros((1, dim), np.float32)
    query[0, 0] = 0.5
    d_corpus, d_q = capi.DeviceArray.from_host(corpus), capi.DeviceArray.from_host(query)
    for flags in (0, capi.SEARCH_FORCE_EXACT_PASS, capi.SEARCH_TEST_TINY_SEGMENTS):
        desc = capi.search_desc(capi.store_desc(d_corpus, n, dim, capi.F32), d_q, 1, k, flags=flags)
        idx, val, _ = capi.search(desc)
        assert idx[0].tolist() == list(range(k)) and np.all(val == 0.5)


@pytest.mark.parametrize("mode", MODES)
def test_monotone_scores_cut_the_running_list(gpu, mode):
    # The last resort sweeps the rows in index order with a running list of keys above its
    # threshold. Scores that ascend with the index append every row, so the list is cut to its
    # width best many times (70,000 rows against lists of at most 12,288 keys); scores that
    # descend fill it once; equal scores keep the lowest indices. Dot products of 0.5 * e0 with
    # rows whose first component is (i + 1) / n are exact in float32.
    capi = gpu
    n, dim, k = 70_000, 64, 100
    corpus = np.zeros((n, dim), np.float32)
    corpus[:, 0] = (np.arange(n, dtype=np.float64) + 1.0) / n
    corpus[:, 1] = 1.0
    queries = np.zeros((3, dim), np.float32)
    queries[0, 0] = 0.5    # ascends with the row index
    queries[1, 0] = -0.5   # descends
    queries[2, 1] = 0.25   # every row scores 0.25
    d_corpus, d_q = capi.DeviceArray.from_host(corpus), capi.DeviceArray.from_host(queries)
    desc = capi.search_desc(capi.store_desc(d_corpus, n, dim, capi.F32), d_q, 3, k, capi.DOT,
                            flags=_flags(capi, mode))
    idx, val = _run(capi, desc, mode)
    ref = oracle.scores_f32(corpus, queries, oracle.DOT)
    ref_idx, ref_val = oracle.topk(ref, k)
    assert np.array_equal(idx, ref_idx) and np.array_equal(val, ref_val)
    assert idx[0].tolist() == list(range(n - 1, n - 1 - k, -1))
    assert idx[1].tolist() == list(range(k)) and idx[2].tolist() == list(range(k))
