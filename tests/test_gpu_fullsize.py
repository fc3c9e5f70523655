"""Parity at the benchmark configurations' full sizes: 1M x 384 float32/float16 (batch 1 and 64),
10M x 768 per-vector int8 (batch 256, k=100), 50M x 1024 binary with a float16 rescore of 1000
candidates (batch 32, k=10) and the 1M-document hybrid BM25 + float16 configuration (batch 16,
k=10). Inputs are generated on the device at their real shapes by the seeded
generator the benchmark uses. The CPU oracle checks every query's top-k against the whole corpus,
copied to the host, at the float, per-vector int8, binary (its Hamming stage) and hybrid
configurations; the sorted and crowded int8 corpora check their flagged queries and a sample. Every
query is also checked for the properties that hold at any size (ids unique and in range, scores
sorted, each returned score equal to the oracle's score of that id)."""

from __future__ import annotations

import numpy as np
import pytest

import bench
import oracle
from helpers import assert_topk_equivalent, float_tolerance

pytestmark = pytest.mark.gpu


def _search(capi, w):
    desc, corpus, queries, keep = bench.build_inputs(capi, w)
    idx, val, flags = capi.search(desc)
    assert not flags.any(), "candidate overflow on a random corpus"
    return idx, val, corpus, queries, keep


def _ranked(idx, val, n):
    for b in range(idx.shape[0]):
        assert len(set(idx[b].tolist())) == idx.shape[1], f"query {b}: repeated id"
        assert ((idx[b] >= 0) & (idx[b] < n)).all(), f"query {b}: id out of range"
        assert np.all(np.diff(val[b].astype(np.float64)) <= 0), f"query {b}: scores not descending"


@pytest.mark.parametrize("workload", ["f32-1m-b1", "f16-1m-b1", "f32-1m-b64", "f16-1m-b64"])
def test_one_million_by_384_float(gpu, workload):
    w = bench.WORKLOADS[workload]
    idx, val, corpus, queries, _ = _search(gpu, w)
    _ranked(idx, val, w["n"])
    decoded = corpus.to_host().astype(np.float32)
    host_q = queries.to_host()
    tol = float_tolerance(host_q, decoded, oracle.COSINE)
    assert_topk_equivalent(idx, val, oracle.scores_f32(decoded, host_q, oracle.COSINE), w["k"], tol)


def test_ten_million_by_768_per_vector_int8(gpu):
    w = bench.WORKLOADS["int8-10m"]
    idx, val, corpus, queries, keep = _search(gpu, w)
    _ranked(idx, val, w["n"])
    codes = corpus.to_host()
    scales = keep["scales"].to_host()
    qcodes, qscales = oracle.quantize_rows_i8(queries.to_host())
    # every query: the reported score of each returned id is the oracle's score, bit for bit
    for b in range(w["batch"]):
        rows = idx[b]
        exact = oracle.scores_i8i8(codes[rows], scales[rows], qcodes[b:b + 1], qscales[b:b + 1])[0]
        assert np.array_equal(val[b], exact), f"query {b}: scores differ from the oracle's"
    # every query: the whole top-100 against a scan of all 10M rows, 32 queries per oracle call
    for b0 in range(0, w["batch"], 32):
        sel = slice(b0, b0 + 32)
        ref = oracle.scores_i8i8(codes, scales, qcodes[sel], qscales[sel])
        assert_topk_equivalent(idx[sel], val[sel], ref, w["k"])
        del ref


def test_ten_million_sorted_rows_are_exact(gpu):
    """The per-vector int8 configuration on a clustered corpus (rows sorted by their first
    coordinate): every result is exact whether or not a query's candidate buffers overflowed
    (overflowed queries take the device's exact fallback inside the same call)."""
    w = bench.WORKLOADS["int8-10m-sorted"]
    desc, corpus, queries, keep = bench.build_inputs(gpu, w)
    idx, val, flags = gpu.search(desc)
    print(f"queries through the exact fallback: {int(np.count_nonzero(flags))} of {w['batch']}", flush=True)
    _ranked(idx, val, w["n"])
    codes = corpus.to_host()
    scales = keep["scales"].to_host()
    assert np.all(np.diff(codes[:, 0].astype(np.int32)) >= 0), "the corpus rows are not sorted"
    qcodes, qscales = oracle.quantize_rows_i8(queries.to_host())
    for b in range(w["batch"]):
        rows = idx[b]
        exact = oracle.scores_i8i8(codes[rows], scales[rows], qcodes[b:b + 1], qscales[b:b + 1])[0]
        assert np.array_equal(val[b], exact), f"query {b}: scores differ from the oracle's"
    sample = [0, 3, 100, 200, 255] + [int(b) for b in np.flatnonzero(flags)[:3]]
    ref = oracle.scores_i8i8(codes, scales, qcodes[sample], qscales[sample])
    assert_topk_equivalent(idx[sample], val[sample], ref, w["k"])


def test_ten_million_crowded_rows_take_the_fallback(gpu):
    """Near-copies of 16 queries crowded into the blocks of one workgroup (bench workload
    int8-10m-hot): those queries' candidates overflow that workgroup's buffers, the merge flags
    them, and the whole-GPU rerun completes them; every result is exact."""
    w = bench.WORKLOADS["int8-10m-hot"]
    desc, corpus, queries, keep = bench.build_inputs(gpu, w)
    idx, val, flags = gpu.search(desc)
    flagged = set(np.flatnonzero(flags).tolist())
    print(f"queries through the exact fallback: {len(flagged)} of {w['batch']}", flush=True)
    assert set(range(w["hot_queries"])) <= flagged, "the crowded queries should take the fallback"
    _ranked(idx, val, w["n"])
    codes = corpus.to_host()
    scales = keep["scales"].to_host()
    qcodes, qscales = oracle.quantize_rows_i8(queries.to_host())
    for b in range(w["batch"]):
        rows = idx[b]
        exact = oracle.scores_i8i8(codes[rows], scales[rows], qcodes[b:b + 1], qscales[b:b + 1])[0]
        assert np.array_equal(val[b], exact), f"query {b}: scores differ from the oracle's"
    hot = set()
    for first in keep["hot_rows"]:
        hot.update(range(first, first + 64))
    for b in range(w["hot_queries"]):
        assert set(idx[b].tolist()) <= hot, f"query {b}: its near-copies should be its top-{w['k']}"
    sample = sorted(flagged | {16, 255})  # every query through the fallback, and two others
    ref = oracle.scores_i8i8(codes, scales, qcodes[sample], qscales[sample])
    assert_topk_equivalent(idx[sample], val[sample], ref, w["k"])


def test_fifty_million_binary_with_fp16_rescore(gpu):
    capi = gpu
    w = bench.WORKLOADS["binary-50m"]
    idx, val, corpus, queries, keep = _search(capi, w)
    _ranked(idx, val, w["n"])
    dim, c, k = w["dim"], w["candidates"], w["k"]
    words = corpus.to_host()
    host_q = queries.to_host()
    half = keep["rescore"]

    def rows_of(ids):
        out = np.empty((len(ids), dim), dtype=np.float16)
        for i, r in enumerate(ids):
            capi.call("zcgvs_memcpy_d2h", out[i].ctypes.data, half.ptr + int(r) * dim * 2, dim * 2, None)
        capi.synchronize()
        return out.astype(np.float32)

    # every query: each returned score is the float16 rescore of that id
    for b in range(w["batch"]):
        got = rows_of(idx[b])
        exact = oracle.rescore(got, host_q[b:b + 1], np.arange(k, dtype=np.int32)[None, :])[0]
        tol = float_tolerance(host_q[b:b + 1], got, oracle.COSINE)[0]
        assert np.all(np.abs(val[b].astype(np.float64) - exact) <= tol), f"query {b}: rescore differs"
    # every query: the Hamming top-1000 stage alone (the same search without the rescore,
    # k = 1000) equals the oracle's top-1000 over all 50M rows, ids and scores bit for bit (8
    # queries per oracle call); then the float16 rescore of those candidates gives the top-10
    sample = list(range(w["batch"]))
    qwords = oracle.pack_binary(host_q)
    stage1 = capi.search_desc(capi.store_desc(corpus, w["n"], dim, capi.BINARY), queries, w["batch"], c,
                              capi.COSINE)
    cand_idx, cand_val, flags = capi.search(stage1)
    assert not flags.any()
    all_cand = np.empty_like(cand_idx)
    for b0 in range(0, w["batch"], 8):
        sel = slice(b0, b0 + 8)
        ref_ids, ref_vals = oracle.topk(oracle.scores_hamming(words, qwords[sel], dim), c)
        assert np.array_equal(cand_idx[sel], ref_ids), f"queries {b0}..: Hamming top-1000 ids differ"
        assert np.array_equal(cand_val[sel], ref_vals), f"queries {b0}..: Hamming top-1000 scores differ"
        all_cand[sel] = ref_ids
    ref_cand = all_cand[sample]
    for i, b in enumerate(sample):
        cand = ref_cand[i]
        rows = rows_of(cand)
        rescored = oracle.rescore(rows, host_q[b:b + 1], np.arange(c, dtype=np.int32)[None, :])
        tol = float_tolerance(host_q[b:b + 1], rows, oracle.COSINE)
        ref_local, ref_val = oracle.topk(rescored, k)
        position = {int(g): j for j, g in enumerate(cand)}
        for r in range(k):
            g, e = int(idx[b, r]), int(cand[ref_local[0, r]])
            assert g in position, f"query {b} rank {r}: id {g} is not a Hamming top-{c} candidate"
            if g != e:
                assert abs(float(rescored[0, position[g]]) - float(ref_val[0, r])) <= (
                    tol[0, position[g]] + tol[0, ref_local[0, r]]), f"query {b} rank {r}: not a near-tie"


def test_one_million_hybrid_bm25_fp16(gpu):
    """The hybrid configuration at its stated size: N = 1,000,000 documents, vocabulary 30,000,
    Poisson(200) lengths, Zipf(1.1) tokens, 8 distinct Zipf terms per query, BM25 k1 = 1.2,
    b = 0.75, fp16 d = 384 cosine, fusion weight 0.5, batch 16, k = 10 - the sliced BM25 sweep over
    sorted postings (245 slices of 4096 documents, head terms with df near N, slice bounds from the
    index's slice table) against the oracle's BM25, maximum and fusion (src/cuda/lexical.cu:17-74,
    tests/cuda/test_lexical.cu:71-93), then the same search with the slice bounds searched per call
    and with the postings scattered (the default, any order), all bit-identical."""
    capi = gpu
    w = bench.WORKLOADS["hybrid-1m"]
    n, k, weight = w["n"], w["k"], w["dense_weight"]
    desc, corpus, queries, keep = bench.build_inputs(capi, w)
    assert desc.flags == capi.SEARCH_SORTED_POSTINGS and desc.lex_slice_table
    idx, val, flags = capi.search(desc)
    assert not flags.any()
    _ranked(idx, val, n)
    index, terms = keep["index"], keep["terms_host"]
    assert index["offsets"][-1] > 100_000_000 and terms.shape == (w["batch"], 8)
    desc.lex_slice_table = None
    idx2, val2, flags = capi.search(desc)
    assert not flags.any()
    assert np.array_equal(idx, idx2) and np.array_equal(val, val2), "slice table and searched bounds differ"
    desc.flags = 0
    idx2, val2, flags = capi.search(desc)
    assert not flags.any()
    assert np.array_equal(idx, idx2) and np.array_equal(val, val2), "sorted sweep and scatter differ"
    decoded = corpus.to_host().astype(np.float32)
    host_q = queries.to_host()
    dense = oracle.scores_f32(decoded, host_q, oracle.COSINE)
    fused = np.empty_like(dense)
    for b in range(w["batch"]):
        lex = oracle.bm25(index["offsets"], index["posting_docs"], index["posting_weights"], terms[b], n)
        assert lex.max() > 0.0
        fused[b] = oracle.fuse(dense[b], lex, oracle.max_positive(lex), weight)
    tol = np.float32(weight) * float_tolerance(host_q, decoded, oracle.COSINE) + 1e-6
    assert_topk_equivalent(idx, val, fused, k, tol)
