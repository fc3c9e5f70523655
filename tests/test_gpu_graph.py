"""A fused search captured into a HIP graph and replayed (zcgvs_graph_* through capi.Graph) gives
bit-identical hits on every replay, with other searches run directly between the replays, as the
reference requires of its graph cache (tests/cpp/test_pipeline.cu:124-157)."""

import numpy as np
import pytest

import oracle
from helpers import normalized

pytestmark = pytest.mark.gpu


def _int8_desc(capi, n, dim, batch, k, seed):
    codes, rs = oracle.quantize_rows_i8(normalized(n, dim, seed))
    queries = normalized(batch, dim, seed + 1)
    store = capi.store_desc(capi.DeviceArray.from_host(codes), n, dim, capi.I8, 1.0, capi.DeviceArray.from_host(rs))
    return capi.search_desc(store, capi.DeviceArray.from_host(queries), batch, k, int8_mode=capi.INT8_PER_VECTOR)


def _f16_desc(capi, n, dim, batch, k, seed):
    rows = oracle.f32_to_f16(normalized(n, dim, seed))
    queries = normalized(batch, dim, seed + 1)
    store = capi.store_desc(capi.DeviceArray.from_host(rows), n, dim, capi.F16)
    return capi.search_desc(store, capi.DeviceArray.from_host(queries), batch, k)


def _f32_desc(capi, n, dim, batch, k, seed):
    corpus = normalized(n, dim, seed)
    queries = normalized(batch, dim, seed + 1)
    store = capi.store_desc(capi.DeviceArray.from_host(corpus), n, dim, capi.F32)
    return capi.search_desc(store, capi.DeviceArray.from_host(queries), batch, k)


def _binary_rescore_desc(capi, n, dim, batch, k, seed):
    rows = normalized(n, dim, seed)
    words, half = oracle.pack_binary(rows), oracle.f32_to_f16(rows)
    queries = normalized(batch, dim, seed + 1)
    return capi.search_desc(capi.store_desc(capi.DeviceArray.from_host(words), n, dim, capi.BINARY),
                            capi.DeviceArray.from_host(queries), batch, k,
                            rescore=capi.store_desc(capi.DeviceArray.from_host(half), n, dim, capi.F16),
                            rescore_candidates=1000)


def _int8_tiny_desc(capi, n, dim, batch, k, seed):
    # two-slot candidate segments: nearly every query is flagged and rerun over the whole corpus
    desc = _int8_desc(capi, n, dim, batch, k, seed)
    desc.flags = capi.SEARCH_TEST_TINY_SEGMENTS
    return desc


def _binary_desc(capi, n, dim, batch, k, seed):
    words = np.random.default_rng(seed).integers(0, 2**32, size=(n, dim // 32), dtype=np.uint32)
    queries = normalized(batch, dim, seed + 1)
    return capi.search_desc(capi.store_desc(capi.DeviceArray.from_host(words), n, dim, capi.BINARY),
                            capi.DeviceArray.from_host(queries), batch, k)


@pytest.mark.parametrize("make,n,dim,batch,k", [
    (_int8_desc, 200_000, 768, 64, 100),   # MFMA scan, several threshold phases
    (_f16_desc, 150_000, 384, 1, 10),      # single pass, one query
    (_f16_desc, 150_000, 384, 16, 10),     # fp16 MFMA scan
    (_f32_desc, 200_000, 384, 64, 10),     # fp32 bf16-split MFMA scan
    (_binary_rescore_desc, 200_000, 1024, 1, 10),  # single pass of 1000 keys, group merges, rescore
    (_int8_desc, 1_000_000, 256, 256, 100),     # sketch plan: sketch, thresholds, one scan, merge
    (_int8_tiny_desc, 1_000_000, 256, 256, 100),  # sketch plan with every query rerun
    (_binary_desc, 2_000_003, 1024, 32, 100),   # binary sketch plan
    (_binary_desc, 2_000_003, 1024, 64, 100),   # two sketch launches, the full scan on the tile kernel
    (_binary_desc, 2_000_003, 1024, 128, 100),  # sketch streamed set by set, full scan on the tile kernel
])
def test_graph_replays_match_direct_calls(gpu, make, n, dim, batch, k):
    capi = gpu
    desc = make(capi, n, dim, batch, k, 31)
    other = make(capi, n // 2, dim, batch, k, 57)
    ref_idx, ref_val, flags = capi.search(desc)
    assert not flags.any() or desc.flags & capi.SEARCH_TEST_TINY_SEGMENTS
    other_idx, other_val, _ = capi.search(other)

    size = capi.search_workspace_bytes(desc)
    workspace = capi.DeviceArray(size, np.uint8)
    out_idx = capi.DeviceArray((batch, k), np.int32)
    out_val = capi.DeviceArray((batch, k), np.float32)
    stream = capi.Stream()
    graph = capi.Graph(stream, lambda: capi.search_topk(desc, workspace, size, out_idx, out_val, stream))
    for replay in range(3):
        graph.launch(stream)
        stream.synchronize()
        np.testing.assert_array_equal(out_idx.to_host(), ref_idx, err_msg=f"replay {replay}")
        np.testing.assert_array_equal(out_val.to_host().view(np.uint32), ref_val.view(np.uint32))
        # direct work of another shape between replays, on its own workspace
        idx, val, _ = capi.search(other)
        np.testing.assert_array_equal(idx, other_idx)
        np.testing.assert_array_equal(val.view(np.uint32), other_val.view(np.uint32))
