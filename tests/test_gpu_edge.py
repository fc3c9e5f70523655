"""Fused search on corpora smaller than one scan tile, on every scan kernel, up to k = corpus size
(a larger k is rejected, as by src/search/searcher.cpp:91-135): the hits must be the oracle's.

Each case runs one dense phase only; it checks the tail handling of the tiles (rows past the
corpus re-read its last row, padded scales) and a merge that keeps every valid key."""

import numpy as np
import pytest

import oracle
from helpers import FLT_MAX, assert_topk_equivalent, float_tolerance, normalized

pytestmark = pytest.mark.gpu


def search(capi, data, n, dim, dtype, queries, k, **kw):
    store = capi.store_desc(capi.DeviceArray.from_host(data), n, dim, dtype, 1.0, kw.pop("row_scales", None))
    desc = capi.search_desc(store, capi.DeviceArray.from_host(queries), queries.shape[0], k, **kw)
    idx, val, flags = capi.search(desc)
    assert not flags.any()
    return idx, val


def assert_hits(idx, val, ref_scores, k, tol=None):
    """Every rank against the oracle; no rank may hold the padding of a missing hit."""
    assert (idx >= 0).all() and (val > -FLT_MAX).all()
    assert_topk_equivalent(idx, val, ref_scores, k, tol)


@pytest.mark.parametrize("n,batch,k", [(1, 1, 1), (37, 1, 37), (37, 8, 37), (100, 8, 10)])
@pytest.mark.parametrize("kind", ["f32", "f16"])
def test_small_float_corpus(gpu, kind, n, batch, k):
    capi = gpu
    dim = 384
    corpus = normalized(n, dim, n + 5)
    queries = normalized(batch, dim, batch + 6)
    if kind == "f32":
        rows, dtype, decoded = corpus, capi.F32, corpus
    else:
        rows = oracle.f32_to_f16(corpus)
        dtype, decoded = capi.F16, rows.astype(np.float32)
    idx, val = search(capi, rows, n, dim, dtype, queries, k)
    ref = oracle.scores_f32(decoded, queries)
    assert_hits(idx, val, ref, k, float_tolerance(queries, decoded, oracle.COSINE))


@pytest.mark.parametrize("n,batch,k", [(1, 1, 1), (37, 1, 37), (37, 16, 37), (65, 16, 64)])
def test_small_per_vector_int8_corpus(gpu, n, batch, k):
    capi = gpu
    dim = 768
    codes, rs = oracle.quantize_rows_i8(normalized(n, dim, n + 7))
    queries = normalized(batch, dim, batch + 8)
    qcodes, qs = oracle.quantize_rows_i8(queries)
    idx, val = search(capi, codes, n, dim, capi.I8, queries, k,
                      row_scales=capi.DeviceArray.from_host(rs), int8_mode=capi.INT8_PER_VECTOR)
    assert_hits(idx, val, oracle.scores_i8i8(codes, rs, qcodes, qs), k)


@pytest.mark.parametrize("n,batch,k", [(1, 1, 1), (37, 1, 37), (37, 8, 37), (300, 8, 10)])
def test_small_binary_corpus(gpu, n, batch, k):
    capi = gpu
    dim = 1024
    words = oracle.pack_binary(normalized(n, dim, n + 9))
    queries = normalized(batch, dim, batch + 10)
    idx, val = search(capi, words, n, dim, capi.BINARY, queries, k)
    assert_hits(idx, val, oracle.scores_hamming(words, oracle.pack_binary(queries), dim), k)
