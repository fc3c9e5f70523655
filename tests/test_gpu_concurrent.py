"""Concurrent searches: several zcgvs_search_topk calls in flight at once on separate streams, each
with its own workspace, must give exactly what the same calls give one at a time.

The library keeps no per-process device state on this path (the caller's workspace holds every
buffer), so searches of different shapes (a batched matrix-core scan, a single-pass scan and a
per-vector int8 scan) launched back to back on three streams may overlap on the GPU in any way.
Their results are compared bit for bit with sequential runs, and the batched float search also
with the CPU oracle.
"""

import numpy as np
import pytest

import oracle
from helpers import assert_topk_equivalent, float_tolerance, normalized

pytestmark = pytest.mark.gpu


def test_searches_on_three_streams_match_sequential_runs(gpu):
    capi = gpu
    n, dim = 120_001, 384
    corpus = normalized(n, dim, 71)
    f16 = oracle.f32_to_f16(corpus)
    codes, scales = oracle.quantize_rows_i8(corpus)
    f16_store = capi.store_desc(capi.DeviceArray.from_host(f16), n, dim, capi.F16)
    d_scales = capi.DeviceArray.from_host(scales)
    i8_store = capi.store_desc(capi.DeviceArray.from_host(codes), n, dim, capi.I8, 1.0, d_scales)

    q64 = normalized(64, dim, 72)
    q1 = normalized(1, dim, 73)
    q16 = normalized(16, dim, 74)
    descs = [
        capi.search_desc(f16_store, capi.DeviceArray.from_host(q64), 64, 10, 0),   # matrix-core float scan
        capi.search_desc(f16_store, capi.DeviceArray.from_host(q1), 1, 50, 1),     # single-pass scan
        capi.search_desc(i8_store, capi.DeviceArray.from_host(q16), 16, 100, 0,
                         int8_mode=capi.INT8_PER_VECTOR),                           # int8 matrix-core scan
    ]

    sequential = []
    for desc in descs:
        idx, val, flags = capi.search(desc)
        assert not flags.any()
        sequential.append((idx, val))
    decoded = f16.astype(np.float32)
    assert_topk_equivalent(sequential[0][0], sequential[0][1], oracle.scores_f32(decoded, q64, 0), 10,
                           float_tolerance(q64, decoded, 0))

    streams = [capi.Stream() for _ in descs]
    sizes = [capi.search_workspace_bytes(d) for d in descs]
    workspaces = [capi.DeviceArray(s, np.uint8) for s in sizes]
    outputs = [(capi.DeviceArray((d.batch, d.k), np.int32), capi.DeviceArray((d.batch, d.k), np.float32))
               for d in descs]
    for _ in range(4):
        for desc, ws, size, (idx, val), stream in zip(descs, workspaces, sizes, outputs, streams):
            capi.search_topk(desc, ws, size, idx, val, stream)
        for round_robin in range(len(descs)):
            # the same searches again, started in another order, before anything is waited on
            j = (round_robin + 1) % len(descs)
            capi.search_topk(descs[j], workspaces[j], sizes[j], outputs[j][0], outputs[j][1], streams[j])
    for stream in streams:
        stream.synchronize()
    capi.synchronize()
    for (idx, val), (ref_idx, ref_val) in zip(outputs, sequential):
        assert np.array_equal(idx.to_host(), ref_idx)
        assert np.array_equal(val.to_host(), ref_val)
