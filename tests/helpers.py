"""Data and comparison helpers shared by the parity tests."""

import numpy as np

import oracle

FLT_MAX = np.finfo(np.float32).max


def normalized(rows, dim, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, dim)).astype(np.float32)
    return oracle.l2_normalize(x)


def float_tolerance(queries, corpus, metric, rel=1e-5):
    """Per-score bound rel * sum_j |q_j c_j| (rel * sum (q-c)^2 for L2): summation-order error of
    a float32 dot product scales with the sum of magnitudes, not with the (possibly ~0) result."""
    q = np.abs(queries.astype(np.float64))
    c = np.abs(corpus.astype(np.float64))
    if metric == oracle.L2:
        mag = (q ** 2).sum(1)[:, None] + (c ** 2).sum(1)[None, :] + 2 * q @ c.T
    else:
        mag = q @ c.T
    return rel * mag + 1e-7


def assert_scores_close(got, expected, tol):
    masked = expected == -FLT_MAX
    assert np.array_equal(got[masked], expected[masked]), "masked scores must be exactly -FLT_MAX"
    err = np.abs(got.astype(np.float64) - expected.astype(np.float64))
    bad = (err > tol) & ~masked
    if bad.any():
        i = np.argwhere(bad)[0]
        raise AssertionError(f"score mismatch at {tuple(i)}: got {got[tuple(i)]} expected "
                             f"{expected[tuple(i)]} tol {np.broadcast_to(tol, got.shape)[tuple(i)]}")


def assert_topk_equivalent(idx, val, ref_scores, k, tol=None):
    """GPU top-k against the oracle's top-k of the oracle scores. Exact for tol=None; for float
    paths a rank may differ only where the oracle's scores of the two ids are within tol."""
    ref_idx, ref_val = oracle.topk(ref_scores, k)
    batch = ref_scores.shape[0]
    for b in range(batch):
        if tol is None:
            assert idx[b].tolist() == ref_idx[b].tolist(), f"query {b}: ids differ"
            assert np.array_equal(val[b], ref_val[b]), f"query {b}: scores differ"
            continue
        t = np.broadcast_to(tol, ref_scores.shape)[b]
        assert len(set(idx[b].tolist())) == k
        for r in range(k):
            g, e = int(idx[b, r]), int(ref_idx[b, r])
            assert 0 <= g < ref_scores.shape[1]
            if g != e:
                assert abs(float(ref_scores[b, g]) - float(ref_scores[b, e])) <= t[g] + t[e], (
                    f"query {b} rank {r}: id {g} vs {e} not a near-tie")
            assert abs(float(val[b, r]) - float(ref_scores[b, g])) <= t[g]
