"""The C++17 host layer (zcgvs_engine: Engine, EmbeddingStore, LexicalIndex over libzcgvs.so) on the
GPU: artifacts written by the NumPy tools load through the C++ readers and search to the oracle's
result; graph replay is bit-identical; a monotone corpus is searched exactly."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from helpers import assert_topk_equivalent, float_tolerance, normalized
from zcgvs_tools import formats, lexical

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def zc(gpu):
    import zcgvs_engine
    return zcgvs_engine


def _engine(zc, tmp_path, corpus, dtype="float32", per_row=False, ids=None, **cfg):
    path = tmp_path / f"corpus.{dtype}{'.rows' if per_row else ''}.zcve"
    formats.write_embeddings(path, corpus, normalized=True, dtype=dtype, per_row_scales=per_row)
    config = zc.EngineConfig()
    config.embeddings_path = str(path)
    if ids is not None:
        meta = tmp_path / "corpus.zcvm"
        formats.write_metadata(meta, ids, [f"passage {j}" for j in range(len(ids))])
        config.metadata_path = str(meta)
    for key, value in cfg.items():
        setattr(config, key, value)
    return zc.Engine(config)


def _options(zc, engine, k, **kw):
    options = engine.default_options()
    options.top_k = k
    options.candidates = k
    for key, value in kw.items():
        setattr(options, key, value)
    return options


def _ids_scores(response):
    ids = np.array([[h.corpus_index for h in hits] for hits in response.results], dtype=np.int64)
    scores = np.array([[h.similarity for h in hits] for hits in response.results], dtype=np.float32)
    return ids, scores


def test_engine_float32_with_metadata(zc, tmp_path):
    n, dim, k = 20_000, 384, 10
    corpus, queries = normalized(n, dim, 1), normalized(5, dim, 2)
    ids = [f"doc-{i}" for i in range(n)]
    engine = _engine(zc, tmp_path, corpus, ids=ids)
    assert (engine.corpus_size, engine.dim, engine.storage_dtype) == (n, dim, "float32")
    response = engine.search_vectors(queries, _options(zc, engine, k))
    got_ids, got_scores = _ids_scores(response)
    ref = oracle.scores_f32(corpus, queries)
    assert_topk_equivalent(got_ids, got_scores, ref, k, float_tolerance(queries, corpus, 0))
    hit = response.results[0][0]
    assert hit.doc_id == ids[hit.corpus_index] and hit.text == f"passage {hit.corpus_index}"
    assert hit.rerank_score == hit.similarity and response.timing.batch == 5
    assert response.timing.search_gpu_ms > 0


def test_engine_per_row_int8_file_is_bit_exact(zc, tmp_path):
    n, dim, k = 30_000, 768, 100
    corpus, queries = normalized(n, dim, 3), normalized(4, dim, 4)
    engine = _engine(zc, tmp_path, corpus, dtype="int8", per_row=True)
    got_ids, got_scores = _ids_scores(engine.search_vectors(queries, _options(zc, engine, k)))
    codes, scales = oracle.quantize_rows_i8(corpus)
    qcodes, qscales = oracle.quantize_rows_i8(queries)
    assert_topk_equivalent(got_ids, got_scores, oracle.scores_i8i8(codes, scales, qcodes, qscales), k)


def test_engine_binary_with_fp16_rescore(zc, tmp_path):
    n, dim, k, c = 40_000, 256, 10, 200
    corpus, queries = normalized(n, dim, 5), normalized(3, dim, 6)
    rescore_path = tmp_path / "rescore.f16.zcve"
    formats.write_embeddings(rescore_path, corpus, normalized=True, dtype="float16")
    engine = _engine(zc, tmp_path, corpus, dtype="binary", rescore_embeddings_path=str(rescore_path),
                     rescore_candidates=c)
    assert engine.has_rescore_store
    got_ids, got_scores = _ids_scores(engine.search_vectors(queries, _options(zc, engine, k)))
    words = oracle.pack_binary(corpus)
    coarse, _ = oracle.topk(oracle.scores_hamming(words, oracle.pack_binary(queries), dim), c)
    store = oracle.f16_to_f32(oracle.f32_to_f16(corpus))
    # exact scores of the coarse candidates, scattered back to corpus positions
    full = np.full((3, n), -np.finfo(np.float32).max, dtype=np.float32)
    rescored = oracle.rescore(store, queries, coarse)
    for q in range(3):
        full[q, coarse[q]] = rescored[q]
    assert_topk_equivalent(got_ids, got_scores, full, k, float_tolerance(queries, store, 0))


def test_engine_hybrid_bm25(zc, tmp_path):
    n, dim, k, vocab = 20_000, 384, 10, 3000
    corpus, queries = normalized(n, dim, 7), normalized(4, dim, 8)
    built = lexical.build_bm25(lexical.synthetic_corpus(n, vocab_size=vocab, mean_length=60, seed=9), vocab)
    lex_path = tmp_path / "lex.zcvl"
    formats.write_lexical_index(lex_path, doc_count=n, vocab_size=vocab, offsets=built["offsets"],
                                posting_docs=built["posting_docs"], posting_weights=built["posting_weights"],
                                k1=1.2, b=0.75, average_doc_length=built["average_doc_length"])
    engine = _engine(zc, tmp_path, corpus, dtype="float16", lexical_index_path=str(lex_path))
    terms = lexical.synthetic_queries(4, terms=8, vocab_size=vocab, seed=10)
    options = _options(zc, engine, k, hybrid=True, dense_weight=0.5)
    got_ids, got_scores = _ids_scores(engine.search_vectors(queries, options, terms.tolist()))
    dense = oracle.scores_f32(oracle.f16_to_f32(oracle.f32_to_f16(corpus)), queries)
    fused = np.empty_like(dense)
    for q in range(4):
        lex = oracle.bm25(built["offsets"], built["posting_docs"], built["posting_weights"], terms[q], n)
        fused[q] = oracle.fuse(dense[q], lex, oracle.max_positive(lex), 0.5)
    assert_topk_equivalent(got_ids, got_scores, fused, k, 0.5 * float_tolerance(queries, corpus, 0, rel=1e-3) + 1e-6)


def test_lexical_index_slice_table(zc, tmp_path):
    # Sorted postings get the slice table at load (one uint32 per term and 4096-document boundary,
    # plus the end); postings out of document order get none and are scattered by the search.
    n, vocab = 20_000, 3000
    built = lexical.build_bm25(lexical.synthetic_corpus(n, vocab_size=vocab, mean_length=60, seed=9), vocab)
    offsets, docs, weights = built["offsets"], built["posting_docs"], built["posting_weights"]
    index = zc.LexicalIndex.from_csr(offsets, docs, weights, n)
    assert index.postings_sorted and index.has_slice_table
    postings = int(offsets[-1])
    assert index.device_bytes == (vocab + 1) * 8 + postings * 8 + vocab * ((n + 4095) // 4096 + 1) * 4
    shuffled = docs.copy()
    lo, hi = int(offsets[0]), int(offsets[1])
    assert hi - lo >= 2
    shuffled[lo:hi] = shuffled[lo:hi][::-1]
    unsorted = zc.LexicalIndex.from_csr(offsets, shuffled, weights, n)
    assert not unsorted.postings_sorted and not unsorted.has_slice_table
    assert unsorted.device_bytes == (vocab + 1) * 8 + postings * 8


def test_graph_replay_is_bit_identical(zc, tmp_path):
    n, dim, k = 50_000, 256, 32
    corpus = normalized(n, dim, 11)
    plain = _engine(zc, tmp_path, corpus)
    graphed = _engine(zc, tmp_path, corpus, use_cuda_graphs=True)
    for seed in (12, 13, 14):
        queries = normalized(6, dim, seed)
        a = plain.search_vectors(queries, _options(zc, plain, k))
        b = graphed.search_vectors(queries, _options(zc, graphed, k))
        assert b.timing.graph_replay and not a.timing.graph_replay
        assert _ids_scores(a)[0].tolist() == _ids_scores(b)[0].tolist()
        assert np.array_equal(_ids_scores(a)[1], _ids_scores(b)[1])
    stats = graphed.stats()
    assert stats.graph_captures == 1 and stats.graph_launches == 3


def test_store_save_load_roundtrip(zc, tmp_path):
    corpus = normalized(1000, 96, 15)
    for dtype, per_row in (("float16", False), ("int8", False), ("binary", False), ("int8", True)):
        store = zc.EmbeddingStore.from_numpy(corpus, dtype, 0.0 if dtype != "int8" else 0.01, True, per_row)
        path = tmp_path / f"saved.{dtype}.{per_row}"
        store.save(str(path))
        rows, normalized_flag, scales = formats.read_embeddings(path, with_row_scales=True)
        assert normalized_flag
        if per_row:
            ref_codes, ref_scales = oracle.quantize_rows_i8(corpus)
            assert np.array_equal(rows, ref_codes) and np.array_equal(scales, ref_scales)
        elif dtype == "float16":
            assert np.array_equal(rows, corpus.astype(np.float16))
        elif dtype == "int8":
            assert np.array_equal(rows, oracle.quantize_i8(corpus, 0.01))
        else:
            assert np.array_equal(rows, oracle.pack_binary(corpus))
        loaded = zc.EmbeddingStore.load(str(path))
        assert (loaded.doc_count, loaded.dim, loaded.dtype, loaded.has_row_scales) == (1000, 96, dtype, per_row)


def test_add_vectors_grows_the_corpus(zc, tmp_path):
    n, dim = 3000, 128
    corpus = normalized(n, dim, 16)
    engine = _engine(zc, tmp_path, corpus, ids=[str(i) for i in range(n)])
    extra = normalized(5, dim, 17)
    engine.add_vectors([f"new-{i}" for i in range(5)], ["x"] * 5, extra)
    assert engine.corpus_size == n + 5
    response = engine.search_vectors(extra, _options(zc, engine, 1))
    assert [hits[0].doc_id for hits in response.results] == [f"new-{i}" for i in range(5)]


def test_monotone_corpus_is_exact(zc, gpu, tmp_path):
    # Scores rise with the row index, so each threshold phase's candidates sit together in the
    # last few blocks: the segments hold a full block each, and a query that still overflowed
    # would be recomputed by the device's exact fallback. Either way the result is exact, through
    # the C ABI and through the Engine.
    capi = gpu
    n, dim, k = 200_000, 64, 10
    theta = (np.pi / 2) * (n - np.arange(n, dtype=np.float64)) / n
    corpus = np.zeros((n, dim), dtype=np.float32)
    corpus[:, 0] = np.cos(theta)
    corpus[:, 1] = np.sin(theta)
    query = np.zeros((1, dim), dtype=np.float32)
    query[0, 0] = 1.0
    d_corpus, d_query = capi.DeviceArray.from_host(corpus), capi.DeviceArray.from_host(query)
    # q = e0 makes every score exactly x_r0 in any summation order, so the comparison is exact;
    # the last ~31 rows round to cos = 1.0f and tie, and ties go to the lowest index
    ref = oracle.scores_f32(corpus, query)
    for flags in (0, capi.SEARCH_TEST_TINY_SEGMENTS, capi.SEARCH_MATERIALIZE):
        desc = capi.search_desc(capi.store_desc(d_corpus, n, dim, capi.F32), d_query, 1, k, flags=flags)
        idx, val, overflow = capi.search(desc)
        assert_topk_equivalent(idx, val, ref, k)
        if flags == capi.SEARCH_TEST_TINY_SEGMENTS:
            assert overflow.any()
    engine = _engine(zc, tmp_path, corpus)
    got_ids, got_scores = _ids_scores(engine.search_vectors(query, _options(zc, engine, k)))
    assert_topk_equivalent(got_ids, got_scores, ref, k)


def test_errors_and_text_queries(zc, tmp_path):
    dim = 64
    corpus = normalized(500, dim, 18)
    engine = _engine(zc, tmp_path, corpus)
    with pytest.raises(ValueError, match="does not match corpus dim"):
        engine.search_vectors(normalized(1, dim + 1, 1), _options(zc, engine, 5))
    strict = _engine(zc, tmp_path, corpus, default_top_k=0)
    options = strict.default_options()
    options.top_k = 0  # falls back to default_top_k, which is 0 here
    with pytest.raises(ValueError, match="top_k must be positive"):
        strict.search_vectors(normalized(1, dim, 1), options)
    with pytest.raises(RuntimeError, match="query embedder"):
        engine.search("hello")

    target = normalized(1, dim, 19)[0]

    class Fixed(zc.QueryEmbedder):
        def embed(self, text):
            return target.tolist()

    engine.set_query_embedder(Fixed())
    hits = engine.search("anything", 3, 3)
    ref_idx, _ = oracle.topk(oracle.scores_f32(corpus, target[None, :]), 3)
    assert [h.corpus_index for h in hits] == ref_idx[0].tolist()
    candidates = engine.retrieve("anything", 3)
    assert [c.corpus_index for c in candidates] == ref_idx[0].tolist()
