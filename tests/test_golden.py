"""Artifact files written by the reference's own tools (tests/golden/, made by
tests/golden/make_reference_fixtures.py with python/zcgvs_tools/formats.py and build_lexical.py of
the reference) against this build's writers, readers and BM25 builder, byte for byte, and the
index's weights against the oracle's BM25 weight. The C++ loaders read the same files on the GPU
(they upload to the device) and write them back unchanged."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from zcgvs_tools import formats, lexical

GOLDEN = Path(__file__).resolve().parent / "golden"
DTYPES = ["float32", "float16", "int8", "binary"]


def _matrix():
    return np.load(GOLDEN / "ref_matrix.npy", allow_pickle=False)


@pytest.mark.parametrize("dtype", DTYPES)
def test_embedding_writer_is_byte_identical(tmp_path, dtype):
    ours = tmp_path / f"ours.{dtype}.zcve"
    formats.write_embeddings(ours, _matrix(), normalized=True, dtype=dtype)
    assert ours.read_bytes() == (GOLDEN / f"ref_{dtype}.zcve").read_bytes()


@pytest.mark.parametrize("dtype", DTYPES)
def test_embedding_reader_decodes_the_reference_file(dtype):
    matrix = _matrix()
    header = formats.read_embedding_header(GOLDEN / f"ref_{dtype}.zcve")
    assert (header["version"], header["doc_count"], header["dim"], header["normalized"]) == (2, 6, 40, True)
    assert header["header_bytes"] == 36  # tests/python/test_formats.py:80
    rows, normalized = formats.read_embeddings(GOLDEN / f"ref_{dtype}.zcve")
    assert normalized
    if dtype == "binary":
        assert np.array_equal(rows, oracle.pack_binary(matrix))
        assert rows[0, 0] & 0b111 == 0b111  # +0.0, -0.0 and 1e-9 all set their bit
    elif dtype == "int8":
        codes, scale = formats.quantize_int8(matrix)
        assert np.array_equal(rows, codes) and np.float32(header["scale"]) == np.float32(scale)
    elif dtype == "float16":
        assert np.array_equal(rows.view(np.uint16), oracle.f32_to_f16(matrix).view(np.uint16))
    else:
        assert np.array_equal(rows.view(np.uint32), matrix.view(np.uint32))


def test_metadata_reader():
    docs = json.loads((GOLDEN / "ref_docs.json").read_text(encoding="utf-8"))
    ids, texts = formats.read_metadata(GOLDEN / "ref_corpus.zcvm")
    assert ids == [f"doc-{i}" for i in range(len(docs))] and texts == docs


def _reference_index():
    return formats.read_lexical_index(GOLDEN / "ref_index.zcvl")


def _tokens():
    return [np.asarray(t, dtype=np.int64) for t in json.loads((GOLDEN / "ref_tokens.json").read_text())]


def test_bm25_builder_matches_the_reference_builder():
    ref = _reference_index()
    vocab = len((GOLDEN / "ref_vocab.txt").read_text(encoding="utf-8").splitlines())
    assert (ref["doc_count"], ref["vocab_size"]) == (6, vocab)
    ours = lexical.build_bm25(_tokens(), vocab, k1=1.2, b=0.75)
    assert np.array_equal(ours["offsets"], ref["offsets"])
    assert np.array_equal(ours["posting_docs"], ref["posting_docs"])
    assert np.array_equal(ours["posting_weights"].view(np.uint32), ref["posting_weights"].view(np.uint32))
    assert np.float32(ours["average_doc_length"]) == np.float32(ref["average_doc_length"])


def test_lexical_writer_is_byte_identical(tmp_path):
    ref = _reference_index()
    ours = tmp_path / "ours.zcvl"
    formats.write_lexical_index(ours, doc_count=ref["doc_count"], vocab_size=ref["vocab_size"],
                                offsets=ref["offsets"], posting_docs=ref["posting_docs"],
                                posting_weights=ref["posting_weights"], k1=ref["k1"], b=ref["b"],
                                average_doc_length=ref["average_doc_length"])
    assert ours.read_bytes() == (GOLDEN / "ref_index.zcvl").read_bytes()


def test_reference_weights_are_the_oracle_bm25_weight():
    ref = _reference_index()
    tokens = _tokens()
    n = ref["doc_count"]
    lengths = [len(t) for t in tokens]
    avgdl = float(np.mean(lengths))
    offsets, docs, weights = ref["offsets"], ref["posting_docs"], ref["posting_weights"]
    for term in range(ref["vocab_size"]):
        df = int(offsets[term + 1] - offsets[term])
        for p in range(offsets[term], offsets[term + 1]):
            doc = int(docs[p])
            tf = int(np.count_nonzero(tokens[doc] == term))
            assert tf > 0
            expected = oracle.bm25_weight(n, df, tf, float(lengths[doc]), avgdl, 1.2, 0.75)
            assert weights[p] == np.float32(expected), (term, doc)
        if df > 1:  # the reference builder writes a term's documents in ascending order
            assert np.all(np.diff(docs[offsets[term]:offsets[term + 1]]) > 0)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
def test_cpp_embedding_loader_roundtrip(gpu, tmp_path, dtype):
    import zcgvs_engine
    store = zcgvs_engine.EmbeddingStore.load(str(GOLDEN / f"ref_{dtype}.zcve"))
    assert (store.doc_count, store.dim, store.dtype, store.normalized) == (6, 40, dtype, True)
    saved = tmp_path / "saved.zcve"
    store.save(str(saved))
    assert saved.read_bytes() == (GOLDEN / f"ref_{dtype}.zcve").read_bytes()


@pytest.mark.gpu
def test_cpp_lexical_loader_roundtrip(gpu, tmp_path):
    import zcgvs_engine
    index = zcgvs_engine.LexicalIndex.load(str(GOLDEN / "ref_index.zcvl"))
    ref = _reference_index()
    assert (index.doc_count, index.vocab_size, index.posting_count) == (6, ref["vocab_size"], ref["nnz"])
    assert (index.k1, index.b) == (pytest.approx(1.2), pytest.approx(0.75))
    saved = tmp_path / "saved.zcvl"
    index.save(str(saved))
    assert saved.read_bytes() == (GOLDEN / "ref_index.zcvl").read_bytes()
