"""Launcher-level parity on the GPU, through the C ABI, against the CPU oracle.

Mirrors the reference's kernel tests: tests/cpp/test_scan_paths.cu (every dispatch path: dims
384/768 chunked, 100 chunked for float32 only, 97 scalar everywhere; dot, dot+mask, L2+mask;
11 queries = one full tile of 8 plus 3), test_topk.cu / test_topk_large.cu, test_quantized.cu,
test_lexical.cu and the conversion kernels.
"""

import numpy as np
import pytest

import oracle
from helpers import FLT_MAX, assert_scores_close, float_tolerance, normalized

pytestmark = pytest.mark.gpu

N = 20000
B = 11
INT8_SCALE = np.float32(1.0 / 127.0)


def stored(capi, x, dtype):
    """(device store, decoded float32 view for the oracle) built with the device converters."""
    d_x = capi.DeviceArray.from_host(x)
    rows, dim = x.shape
    if dtype == capi.F32:
        return d_x, x
    if dtype == capi.F16:
        out = capi.DeviceArray((rows, dim), np.float16)
        capi.launch_convert_f32_to_f16(d_x, out, x.size)
        capi.synchronize()
        host = out.to_host()
        assert np.array_equal(host.view(np.uint16), oracle.f32_to_f16(x).view(np.uint16))
        return out, host.astype(np.float32)
    if dtype == capi.I8:
        out = capi.DeviceArray((rows, dim), np.int8)
        capi.launch_convert_f32_to_i8(d_x, out, x.size, INT8_SCALE)
        capi.synchronize()
        host = out.to_host()
        assert np.array_equal(host, oracle.quantize_i8(x, INT8_SCALE))
        return out, oracle.dequantize_i8(host, INT8_SCALE)
    out = capi.DeviceArray((rows, (dim + 31) // 32), np.uint32)
    capi.launch_pack_binary(d_x, out, rows, dim)
    capi.synchronize()
    host = out.to_host()
    assert np.array_equal(host, oracle.pack_binary(x))
    return out, host


CASES = [(dim, dtype, metric, mask)
         for dim in (384, 768, 100, 97)
         for dtype in (0, 1, 2, 3)
         for metric, mask in ((1, False), (1, True), (2, True))
         if not (dtype == 3 and metric == 2)]


@pytest.mark.parametrize("dim,dtype,metric,use_mask", CASES)
def test_scan_paths(gpu, dim, dtype, metric, use_mask):
    capi = gpu
    corpus = normalized(N, dim, 11 + dim)
    queries = normalized(B, dim, 97 + dim)
    store, decoded = stored(capi, corpus, dtype)
    mask = np.ones(N, dtype=np.uint8)
    mask[::7] = 0
    d_mask = capi.DeviceArray.from_host(mask) if use_mask else None
    scores = capi.DeviceArray((B, N), np.float32)
    if dtype == capi.BINARY:
        qbits = oracle.pack_binary(queries)
        d_q = capi.DeviceArray.from_host(qbits)
        capi.launch_similarity(store, dtype, 1.0, N, dim, d_q, B, d_mask, metric, scores)
        capi.synchronize()
        expected = oracle.scores_hamming(decoded, qbits, dim, mask if use_mask else None)
        assert np.array_equal(scores.to_host(), expected)  # bit-exact
        return
    d_q = capi.DeviceArray.from_host(queries)
    capi.launch_similarity(store, dtype, INT8_SCALE, N, dim, d_q, B, d_mask, metric, scores)
    capi.synchronize()
    expected = oracle.scores_f32(decoded, queries, metric, mask if use_mask else None)
    assert_scores_close(scores.to_host(), expected, float_tolerance(queries, decoded, metric))


@pytest.mark.parametrize("dtype,dim,batch,metric", [
    (0, 384, 4, 0),     # float32, the smallest batch the matrix cores take, cosine
    (0, 256, 64, 1),    # float32 dot, four query groups in one launch
    (1, 512, 130, 0),   # float16, two launches (128 + 2 queries)
    (1, 128, 16, 1),    # float16 dot
])
def test_similarity_batches_on_matrix_cores(gpu, dtype, dim, batch, metric):
    # Unmasked cosine/dot batches of float rows take the float matrix-core scan in its store form
    # (every score written, no keys); 20,003 rows end in a partial tile.
    capi = gpu
    n = 20_003
    corpus = normalized(n, dim, 41 + dim)
    queries = normalized(batch, dim, 43 + batch)
    store, decoded = stored(capi, corpus, dtype)
    scores = capi.DeviceArray((batch, n), np.float32)
    capi.launch_similarity(store, dtype, 1.0, n, dim, capi.DeviceArray.from_host(queries), batch, None, metric,
                           scores)
    capi.synchronize()
    expected = oracle.scores_f32(decoded, queries, metric)
    assert_scores_close(scores.to_host(), expected, float_tolerance(queries, decoded, metric))


@pytest.mark.parametrize("n,batch", [
    (19_968, 8),    # 312 whole tiles of 64 rows: the int8 matrix-core scan in its store form
    (19_968, 300),  # two launches (256 + 44 queries)
    (20_000, 40),   # a partial last tile: the sdot4 scan
])
def test_similarity_i8i8_batches_bit_exact(gpu, n, batch):
    capi = gpu
    corpus = normalized(n, 768, 47)
    queries = normalized(batch, 768, 48)
    codes, rs = oracle.quantize_rows_i8(corpus)
    qcodes, qs = oracle.quantize_rows_i8(queries)
    d_codes, d_rs, d_qcodes, d_qs = (capi.DeviceArray.from_host(a) for a in (codes, rs, qcodes, qs))
    scores = capi.DeviceArray((batch, n), np.float32)
    capi.launch_similarity_i8i8(d_codes, d_rs, n, 768, d_qcodes, d_qs, batch, None, capi.DOT, scores)
    capi.synchronize()
    assert np.array_equal(scores.to_host(), oracle.scores_i8i8(codes, rs, qcodes, qs, None))


def test_similarity_i8i8_bit_exact(gpu):
    capi = gpu
    corpus = normalized(N, 768, 5)
    queries = normalized(B, 768, 6)
    codes, rs = oracle.quantize_rows_i8(corpus)
    qcodes, qs = oracle.quantize_rows_i8(queries)
    # device quantizer must agree bit for bit
    d_x = capi.DeviceArray.from_host(corpus)
    d_codes = capi.DeviceArray((N, 768), np.int8)
    d_rs = capi.DeviceArray(N, np.float32)
    capi.launch_quantize_rows_i8(d_x, N, 768, d_codes, d_rs)
    capi.synchronize()
    assert np.array_equal(d_codes.to_host(), codes)
    assert np.array_equal(d_rs.to_host(), rs)
    mask = (np.arange(N) % 5 != 0).astype(np.uint8)
    scores = capi.DeviceArray((B, N), np.float32)
    d_qcodes, d_qs, d_mask = (capi.DeviceArray.from_host(a) for a in (qcodes, qs, mask))
    capi.launch_similarity_i8i8(d_codes, d_rs, N, 768, d_qcodes, d_qs, B, d_mask, capi.COSINE, scores)
    capi.synchronize()
    assert np.array_equal(scores.to_host(), oracle.scores_i8i8(codes, rs, qcodes, qs, mask))


@pytest.mark.parametrize("n,k,batch,quantized", [
    (5000, 100, 1, False),       # tests/cpp/test_topk.cu
    (1_000_000, 512, 1, False),  # tests/cpp/test_topk_large.cu
    (50000, 1024, 3, True),      # heavy ties: lowest index must win
    (4096, 64, 11, False),       # batched (tests/cpp/test_batched.cu)
    (700, 700, 2, True),         # k == n
    (300_001, 1000, 2, True),    # tile winners merged in groups first; partial last tile; ties
    (1_000_000, 10, 2, False),   # 123 tiles, one merge of their winners
])
def test_topk_exact(gpu, n, k, batch, quantized):
    capi = gpu
    rng = np.random.default_rng(n + k)
    scores = rng.uniform(-1000, 1000, size=(batch, n)).astype(np.float32)
    if quantized:
        scores = np.round(scores / 50).astype(np.float32)
        scores[0, :37] = -0.0
    idx, val = capi.topk(capi.DeviceArray.from_host(scores), k)
    ref_idx, ref_val = oracle.topk(scores, k)
    assert np.array_equal(idx, ref_idx)
    assert np.array_equal(val, ref_val)


def test_topk_argument_errors(gpu):
    capi = gpu
    scores = capi.DeviceArray((1, 100), np.float32)
    out_i = capi.DeviceArray((1, 200), np.int32)
    out_v = capi.DeviceArray((1, 200), np.float32)
    s = [capi.DeviceArray((1, capi.topk_scratch_elements(100, 100)), np.float32) for _ in range(4)]
    with pytest.raises(ValueError, match="exceeds candidate count"):
        capi.launch_topk(scores, 100, 101, 1, out_i, out_v, *s)
    with pytest.raises(ValueError, match="capacity"):
        capi.launch_topk(scores, 5000, 1025, 1, out_i, out_v, *s)


@pytest.mark.parametrize("dtype", [0, 1, 2])
def test_gather_rescore_and_remap(gpu, dtype):
    capi = gpu
    n, dim, batch, count = 3000, 384, 4, 300
    corpus = normalized(n, dim, 77)
    queries = normalized(batch, dim, 78)
    store, decoded = stored(capi, corpus, dtype)
    rng = np.random.default_rng(3)
    cand = rng.integers(-2, n + 2, size=(batch, count)).astype(np.int32)
    values = capi.DeviceArray((batch, count), np.float32)
    d_cand = capi.DeviceArray.from_host(cand)
    d_queries = capi.DeviceArray.from_host(queries)
    capi.launch_gather_rescore(store, dtype, INT8_SCALE, n, dim, d_queries, batch, d_cand, count,
                               capi.COSINE, values)
    capi.synchronize()
    expected = oracle.rescore(decoded, queries, cand)
    tol = np.take_along_axis(float_tolerance(queries, decoded, 0), np.clip(cand, 0, n - 1), 1)
    assert_scores_close(values.to_host(), expected, tol)
    local = rng.integers(-1, count + 1, size=(batch, 10)).astype(np.int32)
    out = capi.DeviceArray((batch, 10), np.int32)
    d_local = capi.DeviceArray.from_host(local)
    capi.launch_remap_indices(d_cand, d_local, count, 10, batch, out)
    capi.synchronize()
    assert np.array_equal(out.to_host(), oracle.remap(cand, local))


def test_gather_rescore_rejects_binary(gpu):
    capi = gpu
    with pytest.raises(ValueError, match="float32, float16 or int8"):
        capi.launch_gather_rescore(1, capi.BINARY, 1.0, 10, 32, 1, 1, 1, 1, 0, 1)


def lexical_index(n, vocab, seed):
    """tests/cpp/test_lexical.cu shape: random postings, one per (term, doc)."""
    rng = np.random.default_rng(seed)
    offsets = [0]
    docs, weights = [], []
    for _ in range(vocab):
        count = int(rng.integers(0, 40))
        docs.extend(rng.choice(n, size=count, replace=False).tolist())
        weights.extend(rng.uniform(0.1, 5.0, size=count).tolist())
        offsets.append(len(docs))
    return (np.array(offsets, np.int64), np.array(docs, np.int32), np.array(weights, np.float32))


def test_lexical_bm25_max_fuse_bit_exact(gpu):
    capi = gpu
    n, vocab = 20000, 3000
    offsets, docs, weights = lexical_index(n, vocab, 41)
    rng = np.random.default_rng(42)
    terms = rng.integers(0, vocab, size=24).astype(np.int32)
    terms[-1] = -1
    dense = rng.uniform(-1, 1, size=n).astype(np.float32)
    d_off, d_docs, d_w = (capi.DeviceArray.from_host(a) for a in (offsets, docs, weights))
    lexical = capi.DeviceArray(n, np.float32, zero=True)
    peak = capi.DeviceArray(1, np.float32, zero=True)
    d_dense = capi.DeviceArray.from_host(dense)
    d_terms = capi.DeviceArray.from_host(terms)
    capi.launch_bm25(d_off, d_docs, d_w, d_terms, terms.size, n, lexical)
    capi.launch_max_positive(lexical, n, peak)
    capi.launch_fuse_scores(d_dense, lexical, peak, 0.6, n)
    capi.synchronize()
    expected_lex = oracle.bm25(offsets, docs, weights, terms, n)
    assert np.array_equal(lexical.to_host(), expected_lex)
    assert peak.to_host()[0] == oracle.max_positive(expected_lex)
    assert np.array_equal(d_dense.to_host(), oracle.fuse(dense, expected_lex, expected_lex.max(), 0.6))


def test_lexical_batched(gpu):
    capi = gpu
    n, vocab, batch, stride = 5000, 500, 5, 8
    offsets, docs, weights = lexical_index(n, vocab, 7)
    rng = np.random.default_rng(8)
    terms = rng.integers(-1, vocab, size=(batch, stride)).astype(np.int32)
    lexical = capi.DeviceArray((batch, n), np.float32, zero=True)
    inputs = [capi.DeviceArray.from_host(a) for a in (offsets, docs, weights, terms)]
    capi.launch_bm25_batched(*inputs, stride, batch, n, lexical)
    capi.synchronize()
    got = lexical.to_host()
    for b in range(batch):
        assert np.array_equal(got[b], oracle.bm25(offsets, docs, weights, terms[b], n))


def test_generate_normalized_rows(gpu):
    capi = gpu
    out = capi.DeviceArray((1000, 384), np.float32)
    capi.generate_normalized(out, 1000, 384, 1234, 0)
    tail = capi.DeviceArray((10, 384), np.float32)
    capi.generate_normalized(tail, 10, 384, 1234, 990)
    capi.synchronize()
    x = out.to_host()
    assert np.allclose(np.linalg.norm(x, axis=1), 1.0, atol=1e-5)
    assert np.array_equal(x[990:], tail.to_host())  # row content depends on (seed, row) only
    assert abs(float(x.mean())) < 0.01
