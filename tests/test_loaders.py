"""The C++ artifact loaders reject malformed files before touching the device (CPU).

Each case corrupts one field of a file the NumPy writer produced and loads it through the C++17
host (zcgvs_engine.EmbeddingStore.load / LexicalIndex.load). The checks mirror the reference's
loaders: src/data/embedding_store.cpp:41-73 (magic, version 0 or unknown, empty matrix, stride
mismatch, quantized rows in version 1) and src/data/lexical_index.cpp:21-47 (magic, version,
empty header, CSR offsets inconsistent with nnz), plus the CSR validation and truncation checks
this build adds. No case reaches a device allocation, so they run without a GPU.
"""

from __future__ import annotations

import struct

import numpy as np
import pytest

from zcgvs_tools import formats


@pytest.fixture(scope="module")
def zc():
    import zcgvs_engine
    return zcgvs_engine


def _zcve(tmp_path, dtype="float32", per_row=False, rows=6, dim=40):
    m = np.random.default_rng(0).standard_normal((rows, dim)).astype(np.float32)
    path = tmp_path / f"m.{dtype}.zcve"
    formats.write_embeddings(path, m, normalized=False, dtype=dtype, per_row_scales=per_row)
    return path, bytearray(path.read_bytes())


def _put(raw: bytearray, offset: int, fmt: str, value) -> None:
    struct.pack_into(fmt, raw, offset, value)


# ZCVE header offsets: magic 0, version 4, flags 8, doc_count 12, dim 20, dtype 24, scale 28,
# row_stride 32; rows start at 36.
@pytest.mark.parametrize("case, edit, message", [
    ("bad magic", lambda r: r.__setitem__(slice(0, 4), b"ZCVX"), "magic mismatch"),
    ("version 0", lambda r: _put(r, 4, "<I", 0), "unsupported embedding file version 0"),
    ("version 4", lambda r: _put(r, 4, "<I", 4), "unsupported embedding file version 4"),
    ("no rows", lambda r: _put(r, 12, "<q", 0), "empty matrix"),
    ("no dims", lambda r: _put(r, 20, "<i", 0), "empty matrix"),
    ("dtype 7", lambda r: _put(r, 24, "<i", 7), "unsupported embedding dtype code 7"),
    ("stride", lambda r: _put(r, 32, "<i", 4 * 40 + 4), "row stride does not match"),
    ("stride 0", lambda r: _put(r, 32, "<i", 0), "row stride does not match"),
    ("truncated", lambda r: r.__delitem__(slice(len(r) - 3, len(r))), "unexpected end of stream"),
    ("header only", lambda r: r.__delitem__(slice(36, len(r))), "unexpected end of stream"),
    ("short header", lambda r: r.__delitem__(slice(30, len(r))), "unexpected end of stream"),
])
def test_embedding_loader_rejects(zc, tmp_path, case, edit, message):
    path, raw = _zcve(tmp_path)
    edit(raw)
    path.write_bytes(bytes(raw))
    with pytest.raises(RuntimeError, match=message):
        zc.EmbeddingStore.load(str(path))


@pytest.mark.parametrize("dtype", ["int8", "binary"])
def test_embedding_loader_rejects_quantized_version_1(zc, tmp_path, dtype):
    path, raw = _zcve(tmp_path, dtype=dtype)
    _put(raw, 4, "<I", 1)
    path.write_bytes(bytes(raw[:28]) + bytes(raw[36:]))  # the v1 header has no scale/stride
    with pytest.raises(RuntimeError, match="quantized embeddings require file version 2"):
        zc.EmbeddingStore.load(str(path))


def test_embedding_loader_rejects_short_row_scales(zc, tmp_path):
    path, raw = _zcve(tmp_path, dtype="int8", per_row=True)
    path.write_bytes(bytes(raw[:-4]))  # one of the six row scales is missing
    with pytest.raises(RuntimeError, match="unexpected end of stream"):
        zc.EmbeddingStore.load(str(path))


def test_embedding_loader_rejects_row_scales_on_float_rows(zc, tmp_path):
    path, raw = _zcve(tmp_path, dtype="float32")
    _put(raw, 4, "<I", 3)
    _put(raw, 8, "<I", formats.FLAG_ROW_SCALES)
    path.write_bytes(bytes(raw) + b"\0" * 24)
    with pytest.raises(RuntimeError, match="per-row scales are defined for int8 rows only"):
        zc.EmbeddingStore.load(str(path))


def test_embedding_loader_missing_file(zc, tmp_path):
    with pytest.raises(RuntimeError, match="cannot open embedding file"):
        zc.EmbeddingStore.load(str(tmp_path / "absent.zcve"))


def _zcvl(tmp_path, offsets, docs, weights, doc_count=10, vocab=4):
    path = tmp_path / "lex.zcvl"
    header = formats._LEX_HEADER.pack(formats.LEXICAL_MAGIC, formats.LEXICAL_VERSION, doc_count, vocab,
                                      len(docs), 1.2, 0.75, 3.0)
    body = (np.asarray(offsets, "<i8").tobytes() + np.asarray(docs, "<i4").tobytes() +
            np.asarray(weights, "<f4").tobytes())
    path.write_bytes(header + body)
    return path


GOOD_OFFSETS = [0, 2, 2, 5, 6]
GOOD_DOCS = [1, 4, 0, 3, 9, 2]
GOOD_WEIGHTS = [0.5, 0.25, 1.0, 2.0, 0.125, 0.75]

# ZCVL header offsets: magic 0, version 4, doc_count 8, vocab 16, nnz 20, k1 28, b 32, avgdl 36;
# term offsets start at 40.


@pytest.mark.parametrize("case, edit, message", [
    ("bad magic", lambda r: r.__setitem__(slice(0, 4), b"ZCVE"), "magic mismatch"),
    ("version 2", lambda r: _put(r, 4, "<I", 2), "unsupported lexical index version 2"),
    ("version 0", lambda r: _put(r, 4, "<I", 0), "unsupported lexical index version 0"),
    ("no docs", lambda r: _put(r, 8, "<q", 0), "empty index"),
    ("no vocab", lambda r: _put(r, 16, "<i", 0), "empty index"),
    ("negative nnz", lambda r: _put(r, 20, "<q", -1), "empty index"),
    ("first offset", lambda r: _put(r, 40, "<q", 1), "offsets are inconsistent with nnz"),
    ("last offset", lambda r: _put(r, 40 + 8 * 4, "<q", 5), "offsets are inconsistent with nnz"),
    ("descending", lambda r: _put(r, 40 + 8 * 2, "<q", 1), "offsets are not ascending"),
    ("doc out of range", lambda r: _put(r, 80 + 4 * 4, "<i", 10), "document out of range"),
    ("negative doc", lambda r: _put(r, 80, "<i", -1), "document out of range"),
    ("truncated", lambda r: r.__delitem__(slice(len(r) - 2, len(r))), "unexpected end of stream"),
])
def test_lexical_loader_rejects(zc, tmp_path, case, edit, message):
    path = _zcvl(tmp_path, GOOD_OFFSETS, GOOD_DOCS, GOOD_WEIGHTS)
    raw = bytearray(path.read_bytes())
    edit(raw)
    path.write_bytes(bytes(raw))
    with pytest.raises(RuntimeError, match=message):
        zc.LexicalIndex.load(str(path))


def test_lexical_from_csr_rejects_bad_arrays(zc):
    with pytest.raises(ValueError, match="vocab \\+ 1 offsets"):
        zc.LexicalIndex.from_csr(np.array([0, 1]), np.array([0, 1], np.int32), np.array([1.0], np.float32), 4)
    with pytest.raises(RuntimeError, match="offsets are not ascending"):
        zc.LexicalIndex.from_csr(np.array([0, 2, 1, 3]), np.array([0, 1, 2], np.int32),
                                 np.ones(3, np.float32), 4)
