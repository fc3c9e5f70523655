"""Fused search (zcgvs_search_topk) parity on the GPU against the CPU oracle.

Shapes follow the benchmark configurations at sizes the oracle finishes in seconds; every case
runs several phases of the scan (the corpus is larger than the first sample), so thresholds,
segments and merges are all exercised. Integer paths (per-vector int8, Hamming) must match the
oracle bit for bit, ids and scores; float paths must match ids except at near-ties within the
float tolerance, and scores within it.
"""

import numpy as np
import pytest

import oracle
from helpers import assert_scores_close, assert_topk_equivalent, float_tolerance, normalized
from zcgvs_tools import lexical

pytestmark = pytest.mark.gpu


def run_search(capi, corpus_dev, n, dim, dtype, queries, k, metric=0, **kw):
    d_q = capi.DeviceArray.from_host(queries)
    store = capi.store_desc(corpus_dev, n, dim, dtype, kw.pop("scale", 1.0), kw.pop("row_scales", None))
    desc = capi.search_desc(store, d_q, queries.shape[0], k, metric, **kw)
    idx, val, flags = capi.search(desc)
    assert not flags.any(), "candidate overflow on a random corpus"
    return idx, val


@pytest.mark.parametrize("n,dim,batch,k,metric", [
    (5183, 384, 1, 10, 0),      # CPU reference configuration (single dense phase)
    (300_000, 384, 1, 10, 0),   # single-query scan, several phases
    (200_000, 384, 13, 100, 2), # L2, partial query tile
])
def test_fused_f32(gpu, n, dim, batch, k, metric):
    capi = gpu
    corpus = normalized(n, dim, 1234)
    queries = normalized(batch, dim, 4321)
    idx, val = run_search(capi, capi.DeviceArray.from_host(corpus), n, dim, capi.F32, queries, k, metric)
    ref = oracle.scores_f32(corpus, queries, metric)
    assert_topk_equivalent(idx, val, ref, k, float_tolerance(queries, corpus, metric))


@pytest.mark.parametrize("batch,k", [(1, 10), (64, 10)])
def test_fused_f16(gpu, batch, k):
    capi = gpu
    n, dim = 250_000, 384
    corpus = normalized(n, dim, 7)
    half = oracle.f32_to_f16(corpus)
    queries = normalized(batch, dim, 8)
    idx, val = run_search(capi, capi.DeviceArray.from_host(half), n, dim, capi.F16, queries, k)
    decoded = half.astype(np.float32)
    ref = oracle.scores_f32(decoded, queries, 0)
    assert_topk_equivalent(idx, val, ref, k, float_tolerance(queries, decoded, 0))


def test_fused_i8_reference_mode_with_mask(gpu):
    capi = gpu
    n, dim, batch, k = 150_000, 768, 5, 50
    corpus = normalized(n, dim, 9)
    scale = np.float32(1.0 / 127.0)
    codes = oracle.quantize_i8(corpus, scale)
    queries = normalized(batch, dim, 10)
    mask = (np.arange(n) % 3 != 1).astype(np.uint8)
    idx, val = run_search(capi, capi.DeviceArray.from_host(codes), n, dim, capi.I8, queries, k,
                          scale=scale, mask=capi.DeviceArray.from_host(mask))
    decoded = oracle.dequantize_i8(codes, scale)
    ref = oracle.scores_f32(decoded, queries, 0, mask)
    assert_topk_equivalent(idx, val, ref, k, float_tolerance(queries, decoded, 0))
    assert np.all(mask[idx] == 1)


@pytest.mark.parametrize("n,dim,batch,k", [
    (120_000, 768, 256, 100),   # per-vector int8 configuration, MFMA path
    (70_001, 384, 37, 10),      # partial last tile, partial query group
    (40_000, 1024, 300, 16),    # two query launches, one n-block per wavefront
    (30_000, 256, 8, 1024),     # k at capacity
    (20_000, 96, 9, 25),        # dim outside the MFMA set: VALU int8 x int8 path
    (300_000, 768, 1, 100),     # single query: VALU int8 x int8 path, several threshold phases
    (50_000, 768, 7, 50),       # below the MFMA batch minimum
    (50_000, 512, 8, 10),       # smallest MFMA batch
])
def test_fused_i8i8_bit_exact(gpu, n, dim, batch, k):
    capi = gpu
    corpus = normalized(n, dim, n + dim)
    queries = normalized(batch, dim, batch + 1)
    codes, rs = oracle.quantize_rows_i8(corpus)
    qcodes, qs = oracle.quantize_rows_i8(queries)
    idx, val = run_search(capi, capi.DeviceArray.from_host(codes), n, dim, capi.I8, queries, k,
                          row_scales=capi.DeviceArray.from_host(rs), int8_mode=capi.INT8_PER_VECTOR)
    ref = oracle.scores_i8i8(codes, rs, qcodes, qs)
    assert_topk_equivalent(idx, val, ref, k)


def test_fused_i8i8_mask(gpu):
    capi = gpu
    n, dim, batch, k = 50_000, 768, 64, 100
    corpus = normalized(n, dim, 3)
    queries = normalized(batch, dim, 4)
    codes, rs = oracle.quantize_rows_i8(corpus)
    qcodes, qs = oracle.quantize_rows_i8(queries)
    mask = (np.arange(n) % 2).astype(np.uint8)
    idx, val = run_search(capi, capi.DeviceArray.from_host(codes), n, dim, capi.I8, queries, k,
                          row_scales=capi.DeviceArray.from_host(rs), int8_mode=capi.INT8_PER_VECTOR,
                          mask=capi.DeviceArray.from_host(mask))
    assert_topk_equivalent(idx, val, oracle.scores_i8i8(codes, rs, qcodes, qs, mask), k)


@pytest.mark.parametrize("n,dim,batch,k", [
    (200_000, 1024, 32, 1000),  # binary configuration shape: massive ties at the top-1000 cut
    (100_000, 384, 3, 10),
    (60_000, 1024, 100, 50),    # more than 32 queries per launch: shared-tile kernel, last set partial
    (80_000, 512, 17, 20),      # one query set, second group of 16 holds a single query
    (50_000, 512, 64, 10),      # 512 dims, two query sets
    (70_000, 1024, 16, 100),    # one query group
    (12_000, 1024, 8, 500),     # few blocks per threshold phase, wide selection: small segments
    (300_000, 1024, 1, 100),    # single query: VALU popcount scan, four row sets per lane, several phases
    (200_000, 512, 2, 50),      # VALU popcount scan, four lanes per 64-byte row
])
def test_fused_hamming_bit_exact(gpu, n, dim, batch, k):
    capi = gpu
    corpus = normalized(n, dim, 5)
    bits = oracle.pack_binary(corpus)
    queries = normalized(batch, dim, 6)
    idx, val = run_search(capi, capi.DeviceArray.from_host(bits), n, dim, capi.BINARY, queries, k)
    ref = oracle.scores_hamming(bits, oracle.pack_binary(queries), dim)
    assert_topk_equivalent(idx, val, ref, k)


def test_fused_odd_dim_takes_materialized_path(gpu):
    capi = gpu
    n, dim, batch, k = 20_000, 97, 4, 20
    corpus = normalized(n, dim, 1)
    half = oracle.f32_to_f16(corpus)
    queries = normalized(batch, dim, 2)
    idx, val = run_search(capi, capi.DeviceArray.from_host(half), n, dim, capi.F16, queries, k)
    decoded = half.astype(np.float32)
    assert_topk_equivalent(idx, val, oracle.scores_f32(decoded, queries, 0), k,
                           float_tolerance(queries, decoded, 0))


def oracle_rescore_pipeline(coarse_scores, store, queries, c, k):
    """Coarse top-C, exact rescore of those rows, final top-k by (exact score, corpus id)."""
    cand, _ = oracle.topk(coarse_scores, c)
    exact = oracle.rescore(store, queries, cand)
    out_idx = np.empty((queries.shape[0], k), np.int32)
    out_val = np.empty((queries.shape[0], k), np.float32)
    for b in range(queries.shape[0]):
        order = sorted(range(c), key=lambda i: (-float(exact[b, i]), int(cand[b, i])))[:k]
        out_idx[b] = cand[b, order]
        out_val[b] = exact[b, order]
    return out_idx, out_val


def test_rescore_lossless_f16_to_f32(gpu):
    # tests/cpp/test_pipeline.cu:80-108: an fp16 coarse pass over 512 candidates cannot lose the
    # true top-10, so the final ids equal the exact CPU top-10.
    capi = gpu
    n, dim, k, c, batch = 8192, 256, 10, 512, 4
    corpus = normalized(n, dim, 31)
    queries = normalized(batch, dim, 33)
    half = capi.DeviceArray.from_host(oracle.f32_to_f16(corpus))
    exact = capi.DeviceArray.from_host(corpus)
    idx, val = run_search(capi, half, n, dim, capi.F16, queries, k,
                          rescore=capi.store_desc(exact, n, dim, capi.F32), rescore_candidates=c)
    ref = oracle.scores_f32(corpus, queries, 0)
    assert_topk_equivalent(idx, val, ref, k, float_tolerance(queries, corpus, 0))


def test_rescore_binary_to_f16(gpu):
    # binary coarse top-C, exact fp16 rescore, final top-k (the binary+rescore configuration)
    capi = gpu
    n, dim, k, c, batch = 100_000, 1024, 10, 1000, 8
    corpus = normalized(n, dim, 50)
    queries = normalized(batch, dim, 51)
    bits = oracle.pack_binary(corpus)
    half = oracle.f32_to_f16(corpus)
    idx, val = run_search(capi, capi.DeviceArray.from_host(bits), n, dim, capi.BINARY, queries, k,
                          rescore=capi.store_desc(capi.DeviceArray.from_host(half), n, dim, capi.F16),
                          rescore_candidates=c)
    coarse = oracle.scores_hamming(bits, oracle.pack_binary(queries), dim)
    decoded = half.astype(np.float32)
    ref_idx, ref_val = oracle_rescore_pipeline(coarse, decoded, queries, c, k)
    tol = float_tolerance(queries, decoded, 0)
    for b in range(batch):
        for r in range(k):
            g, e = int(idx[b, r]), int(ref_idx[b, r])
            if g != e:
                assert abs(float(ref_val[b, r]) - float(val[b, r])) <= tol[b, g] + tol[b, e]
            assert abs(float(val[b, r]) - float(oracle.rescore(decoded, queries[b:b + 1],
                                                               np.array([[g]], np.int32))[0, 0])) <= tol[b, g]


def zipf_lexical_index(n, vocab, seed):
    """Synthetic BM25 index of the hybrid configuration's token model: doc length ~ Poisson(200),
    i.i.d. tokens ~ Zipf(1.1) over ranks 1..V (zcgvs_tools.lexical.synthetic_index, which the
    CPU tests check against the list-based builder and the oracle's BM25 weight)."""
    index = lexical.synthetic_index(n, vocab, seed=seed)
    p = 1.0 / np.arange(1, vocab + 1) ** 1.1
    p /= p.sum()
    return index["offsets"], index["posting_docs"], index["posting_weights"], p


def test_hybrid_bm25_fused(gpu):
    capi = gpu
    n, vocab, dim, batch, k, w = 60_000, 30_000, 384, 16, 10, 0.5
    offsets, docs, weights, p = zipf_lexical_index(n, vocab, 12)
    rng = np.random.default_rng(13)
    terms = np.stack([rng.choice(vocab, size=8, replace=False, p=p) for _ in range(batch)]).astype(np.int32)
    corpus = normalized(n, dim, 14)
    half = oracle.f32_to_f16(corpus)
    queries = normalized(batch, dim, 15)
    idx, val = run_search(capi, capi.DeviceArray.from_host(half), n, dim, capi.F16, queries, k,
                          lex_offsets=capi.DeviceArray.from_host(offsets),
                          lex_docs=capi.DeviceArray.from_host(docs),
                          lex_weights=capi.DeviceArray.from_host(weights), lex_doc_count=n,
                          lex_vocab_size=vocab,
                          query_terms=capi.DeviceArray.from_host(terms), lexical_stride=8,
                          dense_weight=w)
    decoded = half.astype(np.float32)
    dense = oracle.scores_f32(decoded, queries, 0)
    fused = np.empty_like(dense)
    for b in range(batch):
        lex = oracle.bm25(offsets, docs, weights, terms[b], n)
        fused[b] = oracle.fuse(dense[b], lex, oracle.max_positive(lex), w)
    tol = np.float32(w) * float_tolerance(queries, decoded, 0) + 1e-6
    assert_topk_equivalent(idx, val, fused, k, tol)


def test_hybrid_sweep_matches_unsorted_scatter(gpu):
    # With SEARCH_SORTED_POSTINGS the BM25 stage reads document-range slices of sorted postings;
    # by default the postings are scattered slot by slot in any order. Both add a document's
    # weights in slot order, so a shuffled copy of the index gives bit-identical results. Term
    # lists padded with -1 and an out-of-vocabulary id are skipped by both.
    capi = gpu
    n, vocab, dim, batch, k, w = 70_001, 30_000, 384, 12, 10, 0.25
    offsets, docs, weights, p = zipf_lexical_index(n, vocab, 21)
    rng = np.random.default_rng(22)
    terms = np.stack([rng.choice(vocab, size=8, replace=False, p=p) for _ in range(batch)]).astype(np.int32)
    terms[0, 5:] = -1
    terms[1, 7] = vocab + 3
    shuffled_docs, shuffled_weights = docs.copy(), weights.copy()
    for t in range(0, vocab, 7):
        lo, hi = offsets[t], offsets[t + 1]
        order = rng.permutation(hi - lo)
        shuffled_docs[lo:hi] = docs[lo:hi][order]
        shuffled_weights[lo:hi] = weights[lo:hi][order]
    half = oracle.f32_to_f16(normalized(n, dim, 23))
    queries = normalized(batch, dim, 24)
    d_half = capi.DeviceArray.from_host(half)
    d_offsets, d_docs = capi.DeviceArray.from_host(offsets), capi.DeviceArray.from_host(docs)
    table = _slice_table(capi, d_offsets, d_docs, vocab, n)
    results = []
    for doc_array, weight_array, flags, slices in ((docs, weights, capi.SEARCH_SORTED_POSTINGS, None),
                                                   (shuffled_docs, shuffled_weights, 0, None),
                                                   (docs, weights, capi.SEARCH_SORTED_POSTINGS, table)):
        results.append(run_search(capi, d_half, n, dim, capi.F16, queries, k,
                                  lex_offsets=d_offsets, lex_docs=capi.DeviceArray.from_host(doc_array),
                                  lex_weights=capi.DeviceArray.from_host(weight_array), lex_doc_count=n,
                                  lex_vocab_size=vocab, query_terms=capi.DeviceArray.from_host(terms),
                                  lexical_stride=8, dense_weight=w, flags=flags, lex_slice_table=slices))
    for other in results[1:]:
        assert np.array_equal(results[0][0], other[0])
        assert np.array_equal(results[0][1], other[1])
    decoded = half.astype(np.float32)
    dense = oracle.scores_f32(decoded, queries, 0)
    fused = np.empty_like(dense)
    known = np.where(terms < vocab, terms, -1)  # the search skips ids past the vocabulary
    for b in range(batch):
        lex = oracle.bm25(offsets, docs, weights, known[b], n)
        fused[b] = oracle.fuse(dense[b], lex, oracle.max_positive(lex), w)
    tol = np.float32(w) * float_tolerance(queries, decoded, 0) + 1e-6
    assert_topk_equivalent(results[0][0], results[0][1], fused, k, tol)


def _slice_table(capi, d_offsets, d_docs, vocab, doc_count):
    table = capi.DeviceArray(capi.lexical_slice_table_bytes(vocab, doc_count) // 4, np.uint32)
    capi.build_lexical_slice_table(d_offsets, d_docs, vocab, doc_count, table)
    capi.synchronize()
    return table


def test_lexical_slice_table_counts(gpu):
    # Entry (t, c) counts term t's postings below document c * 4096, the last column those below
    # doc_count: numpy's searchsorted over each term's ascending documents gives every entry.
    capi = gpu
    n, vocab = 70_001, 30_000
    offsets, docs, _, _ = zipf_lexical_index(n, vocab, 31)
    stride = (n + 4095) // 4096 + 1
    assert capi.lexical_slice_table_bytes(vocab, n) == vocab * stride * 4
    table = _slice_table(capi, capi.DeviceArray.from_host(offsets), capi.DeviceArray.from_host(docs), vocab, n)
    got = table.to_host().reshape(vocab, stride)
    bounds = np.append(np.arange(stride - 1, dtype=np.int64) * 4096, n)
    expected = np.empty((vocab, stride), np.uint32)
    for t in range(vocab):
        expected[t] = np.searchsorted(docs[offsets[t]:offsets[t + 1]], bounds, side="left")
    assert np.array_equal(got, expected)
    assert got[:, -1].astype(np.int64).sum() == offsets[-1]  # every posting names a document < n


def test_slice_table_of_a_larger_index(gpu):
    # An index over more documents than the corpus scans: its table's slices run to the index's
    # own count, so the corpus's partial last slice takes postings of documents past the corpus,
    # which the BM25 stage skips. Results equal the per-call bounds search and the oracle over
    # the corpus's documents.
    capi = gpu
    n_index, n, vocab, dim, batch, k, w = 70_001, 61_500, 30_000, 256, 6, 10, 0.5
    offsets, docs, weights, p = zipf_lexical_index(n_index, vocab, 41)
    rng = np.random.default_rng(42)
    terms = np.stack([rng.choice(vocab, size=8, replace=False, p=p) for _ in range(batch)]).astype(np.int32)
    half = oracle.f32_to_f16(normalized(n, dim, 43))
    queries = normalized(batch, dim, 44)
    d_offsets, d_docs = capi.DeviceArray.from_host(offsets), capi.DeviceArray.from_host(docs)
    table = _slice_table(capi, d_offsets, d_docs, vocab, n_index)
    d_half = capi.DeviceArray.from_host(half)
    results = [run_search(capi, d_half, n, dim, capi.F16, queries, k, lex_offsets=d_offsets, lex_docs=d_docs,
                          lex_weights=capi.DeviceArray.from_host(weights), lex_doc_count=n_index,
                          lex_vocab_size=vocab, query_terms=capi.DeviceArray.from_host(terms),
                          lexical_stride=8, dense_weight=w, flags=capi.SEARCH_SORTED_POSTINGS,
                          lex_slice_table=slices)
               for slices in (table, None)]
    assert np.array_equal(results[0][0], results[1][0])
    assert np.array_equal(results[0][1], results[1][1])
    decoded = half.astype(np.float32)
    dense = oracle.scores_f32(decoded, queries, 0)
    fused = np.empty_like(dense)
    for b in range(batch):
        lex = oracle.bm25(offsets, docs, weights, terms[b], n)
        fused[b] = oracle.fuse(dense[b], lex, oracle.max_positive(lex), w)
    tol = np.float32(w) * float_tolerance(queries, decoded, 0) + 1e-6
    assert_topk_equivalent(results[0][0], results[0][1], fused, k, tol)


def test_postings_cannot_be_both_sorted_and_unsorted(gpu):
    capi = gpu
    store = capi.store_desc(1 << 20, 5000, 64, capi.F16)
    desc = capi.search_desc(store, 1 << 20, 2, 10, lex_offsets=1 << 20, lex_docs=1 << 20,
                            lex_weights=1 << 20, lex_doc_count=5000, lex_vocab_size=10,
                            query_terms=1 << 20, lexical_stride=4,
                            flags=capi.SEARCH_SORTED_POSTINGS | capi.SEARCH_UNSORTED_POSTINGS)
    with pytest.raises(ValueError, match="both sorted and unsorted"):
        capi.search_workspace_bytes(desc)


@pytest.mark.parametrize("bad,match", [
    (dict(k=0), "k must be positive"),
    (dict(k=2000), "exceeds kernel capacity"),
    (dict(batch=0), "batch must be positive"),
])
def test_search_validation(gpu, bad, match):
    capi = gpu
    store = capi.store_desc(1 << 20, 5000, 64, capi.F32)
    args = dict(batch=1, k=10)
    args.update(bad)
    desc = capi.search_desc(store, 1 << 20, args["batch"], args["k"])
    with pytest.raises(ValueError, match=match):
        capi.search_workspace_bytes(desc)
