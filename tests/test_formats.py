"""Artifact formats and encodings (CPU): the known answers of the reference's
tests/python/test_formats.py, the per-row-scale extension, and cross-checks of the NumPy tools
against the oracle."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from zcgvs_tools import formats, lexical


def _matrix(rows=64, dim=130, seed=3):
    rng = np.random.default_rng(seed)
    m = rng.normal(size=(rows, dim)).astype(np.float32)
    return m / np.linalg.norm(m, axis=1, keepdims=True)


def test_row_strides_known_answers():
    # tests/python/test_formats.py:27-33
    assert formats.row_stride(formats.DTYPE_FLOAT32, 384) == 1536
    assert formats.row_stride(formats.DTYPE_FLOAT16, 384) == 768
    assert formats.row_stride(formats.DTYPE_INT8, 384) == 384
    assert formats.row_stride(formats.DTYPE_BINARY, 384) == 48
    assert formats.row_stride(formats.DTYPE_BINARY, 130) == 20


def test_pack_binary_known_answer_and_padding():
    # tests/python/test_formats.py:36-52
    m = np.full((1, 130), -1.0, dtype=np.float32)
    m[0, 0] = m[0, 33] = m[0, 129] = 1.0
    packed = formats.pack_binary(m)
    assert packed.tolist() == [[1, 2, 0, 0, 2]]
    assert packed[0, 4] >> 2 == 0


def test_pack_binary_matches_oracle_including_signed_zero_and_nan():
    m = _matrix(rows=33, dim=100)
    m[0, :4] = [0.0, -0.0, np.nan, -np.nan]
    assert np.array_equal(formats.pack_binary(m), oracle.pack_binary(m))


def test_int8_matrix_quantization_symmetric_bounded():
    m = _matrix()
    codes, scale = formats.quantize_int8(m)
    assert codes.dtype == np.int8 and codes.min() >= -127 and codes.max() <= 127 and scale > 0
    assert np.max(np.abs(codes.astype(np.float32) * np.float32(scale) - m)) <= scale
    # The file writer divides (rint(x / scale), python/zcgvs_tools/formats.py:85-91); the device
    # converter and the CPU reference multiply by the reciprocal (rint(x * (1 / scale)),
    # src/cuda/convert.cu:25-32, tests/cpp/cpu_reference.hpp:51-62), which the oracle restates.
    # Away from round-half points the two agree to within one code.
    assert np.max(np.abs(codes.astype(np.int32) - oracle.quantize_i8(m, scale).astype(np.int32))) <= 1


def test_int8_division_and_reciprocal_rules_differ_at_a_half_way_point():
    # x / s is exactly 126.5 in float32 and rounds to even (126); x * float32(1 / s) is
    # 126.50001 and rounds to 127. The writer's rule and the device rule are both kept because
    # each is the reference's own rule at its own site.
    x = np.float32(1.5559499)
    s = np.float32(0.0123)
    assert x / s == np.float32(126.5)
    assert np.rint(x / s) == 126.0
    assert oracle.quantize_i8(np.array([x], np.float32), s)[0] == 127
    matrix = np.array([[x, np.float32(127) * s]], np.float32)  # second entry fixes scale = s
    codes, scale = formats.quantize_int8(matrix)
    assert np.float32(scale) == s and codes[0, 0] == 126
    assert oracle.quantize_i8(matrix, scale)[0, 0] == 127


def test_per_row_quantization_matches_the_device_rule():
    m = _matrix(rows=200, dim=96)
    m[5] = 0.0  # all-zero row: scale 1, codes 0
    codes, scales = formats.quantize_rows_int8(m)
    ref_codes, ref_scales = oracle.quantize_rows_i8(m)
    assert np.array_equal(codes, ref_codes)
    assert np.array_equal(scales.view(np.uint32), ref_scales.view(np.uint32))
    assert scales[5] == 1.0 and not codes[5].any()


@pytest.mark.parametrize("dtype", ["float32", "float16", "int8", "binary"])
def test_embedding_roundtrip_every_dtype(tmp_path, dtype):
    m = _matrix()
    path = tmp_path / f"c.{dtype}.zcve"
    formats.write_embeddings(path, m, normalized=True, dtype=dtype)
    header = formats.read_embedding_header(path)
    assert header["version"] == formats.EMBEDDING_VERSION and header["dtype"] == dtype
    assert (header["doc_count"], header["dim"], header["normalized"]) == (64, 130, True)
    assert path.stat().st_size == 36 + header["bytes"]  # v2 header is 36 bytes
    stored, normalized = formats.read_embeddings(path)
    assert normalized is True
    if dtype == "binary":
        assert np.array_equal(stored, formats.pack_binary(m))
    elif dtype == "int8":
        assert np.max(np.abs(stored * np.float32(header["scale"]) - m)) <= header["scale"]
    elif dtype == "float16":
        assert np.array_equal(stored, m.astype(np.float16))
    else:
        assert np.array_equal(stored, m)


def test_storage_size_ratios(tmp_path):
    m = _matrix(rows=256, dim=384)
    sizes = {}
    for dtype in ("float32", "float16", "int8", "binary"):
        path = tmp_path / f"c.{dtype}"
        formats.write_embeddings(path, m, normalized=True, dtype=dtype)
        sizes[dtype] = formats.read_embedding_header(path)["bytes"]
    assert sizes["float32"] // sizes["float16"] == 2
    assert sizes["float32"] // sizes["int8"] == 4
    assert sizes["float32"] // sizes["binary"] == 32


def test_per_row_scale_extension_roundtrip(tmp_path):
    m = _matrix(rows=50, dim=64)
    path = tmp_path / "c.i8rows"
    formats.write_embeddings(path, m, normalized=True, per_row_scales=True)
    header = formats.read_embedding_header(path)
    assert header["version"] == 3 and header["row_scales"] and header["dtype"] == "int8"
    assert path.stat().st_size == 36 + header["bytes"] + 4 * 50
    codes, _, scales = formats.read_embeddings(path, with_row_scales=True)
    ref_codes, ref_scales = oracle.quantize_rows_i8(m)
    assert np.array_equal(codes, ref_codes) and np.array_equal(scales, ref_scales)


def test_quantized_v1_is_rejected(tmp_path):
    import struct
    path = tmp_path / "v1.zcve"
    path.write_bytes(struct.pack("<4sIIqii", b"ZCVE", 1, 0, 1, 4, 2) + b"\0" * 4)
    with pytest.raises(ValueError, match="version 2"):
        formats.read_embedding_header(path)


def test_metadata_roundtrip_utf8(tmp_path):
    ids = ["a", "b-2", "ünïcode"]
    texts = ["first passage", "sécond", "third — with an em dash"]
    path = tmp_path / "m.zcvm"
    formats.write_metadata(path, ids, texts)
    assert formats.read_metadata(path) == (ids, texts)


def test_lexical_roundtrip_and_bm25_weights(tmp_path):
    docs = lexical.synthetic_corpus(300, vocab_size=500, mean_length=40, seed=5)
    built = lexical.build_bm25(docs, 500)
    offsets, pdocs, pweights = built["offsets"], built["posting_docs"], built["posting_weights"]
    assert offsets[0] == 0 and offsets[-1] == pdocs.size and np.all(np.diff(offsets) >= 0)
    # every posting weight is the oracle's BM25 formula (float64, cast to float32)
    df = np.diff(offsets)
    lengths = np.array([len(d) for d in docs])
    for term in (0, 1, 7, 123):
        for j in range(offsets[term], offsets[term + 1]):
            d = pdocs[j]
            tf = int(np.count_nonzero(np.asarray(docs[d]) == term))
            expected = np.float32(oracle.bm25_weight(300, int(df[term]), tf, lengths[d], built["average_doc_length"]))
            assert pweights[j] == expected
        assert np.all(np.diff(pdocs[offsets[term]:offsets[term + 1]]) > 0)
    path = tmp_path / "lex.zcvl"
    formats.write_lexical_index(path, doc_count=300, vocab_size=500, offsets=offsets, posting_docs=pdocs,
                                posting_weights=pweights, k1=1.2, b=0.75,
                                average_doc_length=built["average_doc_length"])
    back = formats.read_lexical_index(path)
    assert back["nnz"] == pdocs.size and np.array_equal(back["offsets"], offsets)
    assert np.array_equal(back["posting_docs"], pdocs) and np.array_equal(back["posting_weights"], pweights)


def test_synthetic_queries_have_distinct_terms():
    q = lexical.synthetic_queries(16, terms=8, vocab_size=30_000)
    assert q.shape == (16, 8)
    assert all(len(set(row.tolist())) == 8 for row in q)
