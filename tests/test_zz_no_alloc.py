"""zcgvs_search_topk_noalloc (workspace in the library's static device array) against
zcgvs_search_topk (caller workspace), through the C ABI: two calls in a row on each path, the
second with a smaller input, bit-identical ids and scores; the entry point captured into a HIP
graph and replayed gives the same result on every replay; a search whose workspace exceeds the
static array is rejected."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from helpers import normalized

pytestmark = pytest.mark.gpu


def _pair(capi, desc):
    """(ids, scores) of the workspace entry point and of the no-allocation one."""
    expected = capi.search(desc)
    idx = capi.DeviceArray((desc.batch, desc.k), np.int32)
    val = capi.DeviceArray((desc.batch, desc.k), np.float32)
    capi.call("zcgvs_search_topk_noalloc", capi.ctypes.byref(desc), idx.ptr, val.ptr, None)
    capi.synchronize()
    return expected, (idx.to_host(), val.to_host())


def _int8_case(capi, n, batch, seed):
    dim, k = 768, 100
    codes, scales = oracle.quantize_rows_i8(normalized(n, dim, seed))
    queries = normalized(batch, dim, seed + 1)
    d_codes, d_scales, d_queries = (capi.DeviceArray.from_host(a) for a in (codes, scales, queries))
    desc = capi.search_desc(capi.store_desc(d_codes, n, dim, capi.I8, 1.0, d_scales), d_queries, batch, k,
                            capi.COSINE, int8_mode=capi.INT8_PER_VECTOR)
    qcodes, qscales = oracle.quantize_rows_i8(queries)
    ref = oracle.topk(oracle.scores_i8i8(codes, scales, qcodes, qscales), k)
    return desc, ref, (d_codes, d_scales, d_queries)


def _float_case(capi, n, batch, seed):
    dim, k = 384, 10
    corpus = normalized(n, dim, seed)
    queries = normalized(batch, dim, seed + 1)
    d_corpus, d_queries = capi.DeviceArray.from_host(corpus), capi.DeviceArray.from_host(queries)
    desc = capi.search_desc(capi.store_desc(d_corpus, n, dim, capi.F32), d_queries, batch, k, capi.COSINE)
    return desc, None, (d_corpus, d_queries)


def test_static_scratch_size(gpu):
    assert gpu.library().zcgvs_static_scratch_bytes() == 64 << 20


@pytest.mark.parametrize("case", ["int8", "float32", "float32-few"])
def test_noalloc_matches_the_workspace_entry_point(gpu, case):
    capi = gpu
    build = _int8_case if case == "int8" else _float_case
    # two calls in a row, the second smaller: the array keeps the first call's contents (the
    # few-query case takes the single pass)
    sizes = ((300_000, 3, 31), (70_001, 1, 41)) if case == "float32-few" else ((300_000, 48, 11), (70_001, 9, 21))
    for n, batch, seed in sizes:
        desc, ref, _keep = build(capi, n, batch, seed)
        assert capi.search_workspace_bytes(desc) <= 64 << 20
        (exp_idx, exp_val, flags), (got_idx, got_val) = _pair(capi, desc)
        assert not flags.any()
        assert np.array_equal(got_idx, exp_idx), f"{case} n={n}: ids differ"
        assert np.array_equal(got_val, exp_val), f"{case} n={n}: scores differ"
        if ref is not None:
            assert np.array_equal(got_idx, ref[0]) and np.array_equal(got_val, ref[1])


def test_noalloc_rejects_a_search_beyond_the_static_scratch(gpu):
    capi = gpu
    n, dim, batch = 2_000_000, 128, 64
    store = capi.store_desc(1 << 20, n, dim, capi.F32)
    desc = capi.search_desc(store, 1 << 20, batch, 10, capi.COSINE, flags=capi.SEARCH_MATERIALIZE)
    assert capi.search_workspace_bytes(desc) > 64 << 20  # a [64, 2M] score matrix
    with pytest.raises(ValueError, match="static scratch"):
        capi.call("zcgvs_search_topk_noalloc", capi.ctypes.byref(desc), 1 << 20, 1 << 20, None)


def test_noalloc_captured_in_a_graph(gpu):
    """Captured once (zcgvs_graph_begin_capture resolves the static scratch first), replayed
    three times with other searches in between; every replay equals the direct call."""
    capi = gpu
    desc, ref, _keep = _int8_case(capi, 120_000, 16, 51)
    other, _, _keep2 = _float_case(capi, 90_000, 5, 61)
    (exp_idx, exp_val, _), _ = _pair(capi, desc)
    assert np.array_equal(exp_idx, ref[0]) and np.array_equal(exp_val, ref[1])
    idx = capi.DeviceArray((desc.batch, desc.k), np.int32)
    val = capi.DeviceArray((desc.batch, desc.k), np.float32)
    stream = capi.Stream()
    graph = capi.Graph(stream, lambda: capi.call("zcgvs_search_topk_noalloc", capi.ctypes.byref(desc), idx.ptr,
                                                 val.ptr, stream.handle))
    for replay in range(3):
        capi.call("zcgvs_memset", idx.ptr, 0, idx.nbytes, None)
        capi.synchronize()
        graph.launch(stream)
        stream.synchronize()
        assert np.array_equal(idx.to_host(), exp_idx), f"replay {replay}: ids differ"
        assert np.array_equal(val.to_host(), exp_val), f"replay {replay}: scores differ"
        # eager work on the same static scratch between replays
        capi.call("zcgvs_search_topk_noalloc", capi.ctypes.byref(other), idx.ptr, val.ptr, None)
        capi.synchronize()
