"""Batched float32 / float16 searches (the matrix-core scan) against the CPU oracle.

Batches of 4 or more queries over float32 or float16 rows of 128, 256, 384 or 512 dims take the
MFMA scan; launches of 32 to 128 queries over float32 rows of 256 or 384 dims take its bf16
three-part split form. These cases cover every such row size, partial query groups (17, 33, 40),
a batch over two launches (130: a split launch of 128 and a float32 launch of 2), a partial last
tile (n not a multiple of the tile rows), k = 1 and k = 100, both metrics, query magnitudes far
from 1 (the float16 path rescales each query by a power of two before splitting it), and rows
whose components span thirty binary orders of magnitude (every part of the bf16 split matters). Ids must match the oracle's except at near-ties within the float32
tolerance, and every score must be within it."""

import numpy as np
import pytest

import oracle
from helpers import assert_topk_equivalent, float_tolerance, normalized

pytestmark = pytest.mark.gpu


def search(capi, rows, dtype, queries, k, metric):
    n, dim = rows.shape
    store = capi.store_desc(capi.DeviceArray.from_host(rows), n, dim, dtype)
    desc = capi.search_desc(store, capi.DeviceArray.from_host(queries), queries.shape[0], k, metric)
    idx, val, flags = capi.search(desc)
    assert not flags.any(), "candidate overflow on a random corpus"
    return idx, val


CASES = [
    # kind, n, dim, batch, k, metric, query scale
    ("f32", 60_013, 128, 17, 10, 0, 1.0),
    ("f32", 60_013, 256, 17, 10, 1, 1.0),
    ("f32", 100_003, 384, 4, 10, 0, 1.0),
    ("f32", 100_003, 384, 64, 100, 1, 1.0),
    ("f32", 100_003, 384, 130, 10, 0, 1.0),
    ("f32", 60_013, 512, 33, 1, 0, 1.0),
    ("f32", 60_013, 256, 32, 10, 0, 1.0),
    ("f32", 100_003, 384, 40, 10, 1, 1000.0),
    ("f32", 100_003, 384, 48, 10, 0, 1e-3),
    ("f16", 60_013, 128, 17, 10, 0, 1.0),
    ("f16", 60_013, 256, 17, 10, 1, 1.0),
    ("f16", 100_003, 384, 4, 10, 0, 1.0),
    ("f16", 100_003, 384, 64, 100, 1, 1.0),
    ("f16", 100_003, 384, 130, 10, 0, 1.0),
    ("f16", 60_013, 512, 33, 1, 0, 1.0),
    ("f16", 100_003, 384, 16, 10, 1, 1000.0),
    ("f16", 100_003, 384, 16, 10, 1, 1e-3),
]


@pytest.mark.parametrize("kind,n,dim,batch,k,metric,qscale", CASES)
def test_batched_float_scan(gpu, kind, n, dim, batch, k, metric, qscale):
    capi = gpu
    corpus = normalized(n, dim, 100 + dim)
    queries = (normalized(batch, dim, 200 + batch) * np.float32(qscale)).astype(np.float32)
    if kind == "f32":
        rows, dtype, decoded = corpus, capi.F32, corpus
    else:
        rows = oracle.f32_to_f16(corpus)
        dtype, decoded = capi.F16, rows.astype(np.float32)
    idx, val = search(capi, rows, dtype, queries, k, metric)
    ref = oracle.scores_f32(decoded, queries, metric)
    assert_topk_equivalent(idx, val, ref, k, float_tolerance(queries, decoded, metric))


def test_batched_float_scan_ties(gpu):
    # Row i repeats row i % 1000, so each class of 40 identical rows ties exactly on any path:
    # within a class the result must hold its lowest ids, in ascending order.
    capi = gpu
    n, dim, batch, k = 40_000, 384, 8, 50
    base = normalized(1000, dim, 5)
    corpus = base[np.arange(n) % 1000]
    queries = normalized(batch, dim, 6)
    for kind in ("f32", "f16"):
        rows = corpus if kind == "f32" else oracle.f32_to_f16(corpus)
        dtype = capi.F32 if kind == "f32" else capi.F16
        decoded = rows.astype(np.float32)
        idx, val = search(capi, rows, dtype, queries, k, 0)
        assert_topk_equivalent(idx, val, oracle.scores_f32(decoded, queries, 0), k,
                               float_tolerance(queries, decoded, 0))
        for b in range(batch):
            classes = idx[b] % 1000
            for c in np.unique(classes):
                members = idx[b][classes == c]
                lowest = c + 1000 * np.arange(len(members))
                assert np.array_equal(members, lowest), f"{kind} query {b}: class {c} ids {members}"


@pytest.mark.parametrize("dim,batch", [(256, 64), (384, 96)])
def test_split_scan_wide_dynamic_range(gpu, dim, batch):
    """Rows and queries whose components are scaled by 2^-30 .. 2^0 (per component): the bf16
    split must carry the low parts of every value, or the scores miss the float32 tolerance."""
    capi = gpu
    n, k = 80_021, 20
    rng = np.random.default_rng(dim + batch)
    corpus = normalized(n, dim, 300 + dim) * np.exp2(rng.integers(-30, 1, size=(n, dim))).astype(np.float32)
    queries = normalized(batch, dim, 400 + dim) * np.exp2(rng.integers(-30, 1, size=(batch, dim))).astype(np.float32)
    corpus, queries = corpus.astype(np.float32), queries.astype(np.float32)
    idx, val = search(capi, corpus, capi.F32, queries, k, 1)
    ref = oracle.scores_f32(corpus, queries, 1)
    assert_topk_equivalent(idx, val, ref, k, float_tolerance(queries, corpus, 1))


def test_non_finite_rows_depend_on_the_scan(gpu):
    """A float32 row with an infinite component: the bf16 split scan (32-128 queries of 256 or 384
    dims per launch) scores it NaN, which ranks last; the float32 scans follow the IEEE sum, so for
    a query whose matching component is positive it scores +inf and ranks first. This pins the
    documented difference (the reference defines no order for non-finite scores)."""
    capi = gpu
    n, dim, k = 40_000, 384, 10
    corpus = normalized(n, dim, 501)
    corpus[7, 5] = np.float32(np.inf)
    queries = normalized(32, dim, 502)
    queries[:, 5] = np.abs(queries[:, 5]) + np.float32(0.01)  # the inf component meets a positive one
    idx, val = search(capi, corpus, capi.F32, queries, k, 1)  # 32 queries: the split scan
    assert not (idx == 7).any(), "the split scan should rank the non-finite row last"
    one_idx, one_val = search(capi, corpus, capi.F32, queries[:1], k, 1)  # one query: float32 sums
    assert one_idx[0, 0] == 7 and np.isinf(one_val[0, 0]) and one_val[0, 0] > 0
    # the finite rows agree with the oracle either way
    finite = np.ones(n, dtype=bool)
    finite[7] = False
    ref = oracle.scores_f32(corpus[finite], queries, 1)
    remap = np.flatnonzero(finite)
    ref_idx, _ = oracle.topk(ref, k)
    tol = float_tolerance(queries, corpus[finite], 1)
    for b in range(queries.shape[0]):
        for r in range(k):
            g, e = int(idx[b, r]), int(remap[ref_idx[b, r]])
            if g != e:
                gi = int(np.flatnonzero(remap == g)[0])
                assert abs(float(ref[b, gi]) - float(ref[b, ref_idx[b, r]])) <= tol[b, gi] + tol[b, ref_idx[b, r]]
