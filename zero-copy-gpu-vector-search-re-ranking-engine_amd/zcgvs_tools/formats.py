"""ZCVE / ZCVM / ZCVL readers and writers and the storage encodings, NumPy only.

Byte layouts follow include/zcgvs/data/binary_format.hpp:12-62 of the reference (little-endian),
and the function names follow python/zcgvs_tools/formats.py, so artifacts move between the two
builds. Version 3 of ZCVE is this build's extension: int8 rows with one scale per row (flags bit
1), the scales stored as [doc_count] float32 after the rows.
"""

from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

EMBEDDING_MAGIC = b"ZCVE"
METADATA_MAGIC = b"ZCVM"
LEXICAL_MAGIC = b"ZCVL"
EMBEDDING_VERSION = 2
EMBEDDING_ROW_SCALE_VERSION = 3
METADATA_VERSION = 1
LEXICAL_VERSION = 1

FLAG_NORMALIZED = 1 << 0
FLAG_ROW_SCALES = 1 << 1

DTYPE_FLOAT32, DTYPE_FLOAT16, DTYPE_INT8, DTYPE_BINARY = 0, 1, 2, 3
DTYPE_NAMES = {"float32": DTYPE_FLOAT32, "float16": DTYPE_FLOAT16, "int8": DTYPE_INT8, "binary": DTYPE_BINARY}
DTYPE_CODES = {code: name for name, code in DTYPE_NAMES.items()}
_NUMPY = {DTYPE_FLOAT32: np.float32, DTYPE_FLOAT16: np.float16, DTYPE_INT8: np.int8, DTYPE_BINARY: np.uint32}

_HEADER_V1 = struct.Struct("<4sIIqii")      # magic, version, flags, doc_count, dim, dtype
_HEADER_V2_TAIL = struct.Struct("<fi")      # scale, row_stride


def binary_words(dim: int) -> int:
    """u32 words per sign-packed row."""
    return (dim + 31) // 32


def row_stride(dtype_code: int, dim: int) -> int:
    """Bytes per stored row."""
    per = {DTYPE_FLOAT32: 4 * dim, DTYPE_FLOAT16: 2 * dim, DTYPE_INT8: dim, DTYPE_BINARY: 4 * binary_words(dim)}
    if dtype_code not in per:
        raise ValueError(f"unknown dtype code {dtype_code}")
    return per[dtype_code]


def pack_binary(matrix: np.ndarray) -> np.ndarray:
    """Sign bits, bit b of word w = dimension 32 w + b, set when the value is >= 0 (so -0.0 sets
    it and NaN does not); padding bits past dim are zero."""
    matrix = np.ascontiguousarray(matrix, dtype=np.float32)
    rows, dim = matrix.shape
    words = binary_words(dim)
    bits = np.zeros((rows, words * 32), dtype=np.uint8)
    bits[:, :dim] = matrix >= 0.0
    # little bit order inside each byte, little-endian bytes inside each word
    return np.packbits(bits, axis=1, bitorder="little").view("<u4").reshape(rows, words).astype(np.uint32)


def quantize_int8(matrix: np.ndarray) -> tuple[np.ndarray, float]:
    """One scale for the whole matrix: scale = max|x| / 127 (1.0 for an all-zero matrix),
    codes = rint(x / float32(scale)) clipped to +-127 (round half to even)."""
    matrix = np.ascontiguousarray(matrix, dtype=np.float32)
    peak = float(np.abs(matrix).max()) if matrix.size else 0.0
    scale = peak / 127.0 if peak > 0.0 else 1.0
    codes = np.clip(np.rint(matrix / np.float32(scale)), -127, 127).astype(np.int8)
    return codes, scale


def quantize_rows_int8(matrix: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """One scale per row: s = float32(max|x_row|) / 127 in float32 (1.0 for an all-zero row),
    codes = rint(x * float32(1 / s)) clipped to +-127 - the rule the device quantizer applies."""
    matrix = np.ascontiguousarray(matrix, dtype=np.float32)
    peak = np.abs(matrix).max(axis=1).astype(np.float32)
    scales = np.where(peak > 0, peak / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    inverse = (np.float32(1.0) / scales).astype(np.float32)
    codes = np.clip(np.rint(matrix * inverse[:, None]), -127, 127).astype(np.int8)
    return codes, scales


def encode_matrix(matrix: np.ndarray, dtype: str) -> tuple[np.ndarray, int, float]:
    """(storage array, dtype code, matrix-wide scale) for a float32 matrix."""
    if dtype not in DTYPE_NAMES:
        raise ValueError(f"unknown storage dtype '{dtype}'")
    code = DTYPE_NAMES[dtype]
    if code == DTYPE_FLOAT32:
        return np.ascontiguousarray(matrix, dtype=np.float32), code, 1.0
    if code == DTYPE_FLOAT16:
        return np.ascontiguousarray(matrix, dtype=np.float16), code, 1.0
    if code == DTYPE_INT8:
        codes, scale = quantize_int8(matrix)
        return codes, code, scale
    return pack_binary(matrix), code, 1.0


def write_embeddings(path: str | Path, matrix: np.ndarray, normalized: bool, dtype: str | None = None,
                     per_row_scales: bool = False) -> None:
    """Writes ZCVE version 2 (version 3 for int8 with per-row scales)."""
    matrix = np.asarray(matrix)
    if matrix.ndim != 2:
        raise ValueError("embedding matrix must be 2-D")
    doc_count, dim = matrix.shape
    if per_row_scales:
        storage, row_scales = quantize_rows_int8(matrix)
        code, scale, version = DTYPE_INT8, 1.0, EMBEDDING_ROW_SCALE_VERSION
    else:
        storage, code, scale = encode_matrix(matrix, dtype or "float32")
        row_scales, version = None, EMBEDDING_VERSION
    flags = (FLAG_NORMALIZED if normalized else 0) | (FLAG_ROW_SCALES if row_scales is not None else 0)
    with open(path, "wb") as out:
        out.write(_HEADER_V1.pack(EMBEDDING_MAGIC, version, flags, doc_count, dim, code))
        out.write(_HEADER_V2_TAIL.pack(scale, row_stride(code, dim)))
        out.write(np.ascontiguousarray(storage).astype(np.dtype(_NUMPY[code]).newbyteorder("<"), copy=False).tobytes())
        if row_scales is not None:
            out.write(row_scales.astype("<f4").tobytes())


def read_embedding_header(path: str | Path) -> dict:
    with open(path, "rb") as f:
        raw = f.read(_HEADER_V1.size)
        if len(raw) < _HEADER_V1.size:
            raise ValueError("truncated embedding header")
        magic, version, flags, doc_count, dim, code = _HEADER_V1.unpack(raw)
        if magic != EMBEDDING_MAGIC:
            raise ValueError("not a ZCVE embedding file")
        if version < 1 or version > EMBEDDING_ROW_SCALE_VERSION:
            raise ValueError(f"unsupported embedding file version {version}")
        if code not in DTYPE_CODES:
            raise ValueError(f"unknown dtype code {code}")
        scale, stride = 1.0, row_stride(code, dim)
        header_bytes = _HEADER_V1.size
        if version >= 2:
            scale, recorded = _HEADER_V2_TAIL.unpack(f.read(_HEADER_V2_TAIL.size))
            if recorded != stride:
                raise ValueError("row stride does not match dtype and dim")
            header_bytes += _HEADER_V2_TAIL.size
        elif code in (DTYPE_INT8, DTYPE_BINARY):
            raise ValueError("quantized embeddings require file version 2")
    return {"version": version, "flags": flags, "normalized": bool(flags & FLAG_NORMALIZED),
            "row_scales": bool(version >= 3 and flags & FLAG_ROW_SCALES), "doc_count": doc_count, "dim": dim,
            "dtype_code": code, "dtype": DTYPE_CODES[code], "scale": float(scale), "row_stride": stride,
            "bytes": doc_count * stride, "header_bytes": header_bytes}


def read_embeddings(path: str | Path, with_row_scales: bool = False):
    """(stored rows, normalized) - or (rows, normalized, row scales) with with_row_scales."""
    header = read_embedding_header(path)
    code, n, dim = header["dtype_code"], header["doc_count"], header["dim"]
    width = binary_words(dim) if code == DTYPE_BINARY else dim
    rows = np.fromfile(path, dtype=np.dtype(_NUMPY[code]).newbyteorder("<"), count=n * width,
                       offset=header["header_bytes"]).reshape(n, width)
    rows = rows.astype(_NUMPY[code], copy=False)
    if not with_row_scales:
        return rows, header["normalized"]
    scales = None
    if header["row_scales"]:
        scales = np.fromfile(path, dtype="<f4", count=n, offset=header["header_bytes"] + header["bytes"])
        scales = scales.astype(np.float32)
    return rows, header["normalized"], scales


def write_metadata(path: str | Path, doc_ids: list[str], texts: list[str]) -> None:
    if len(doc_ids) != len(texts):
        raise ValueError("doc_ids and texts must have equal length")
    with open(path, "wb") as out:
        out.write(struct.pack("<4sIq", METADATA_MAGIC, METADATA_VERSION, len(doc_ids)))
        for doc_id, text in zip(doc_ids, texts):
            for field in (doc_id.encode("utf-8"), text.encode("utf-8")):
                out.write(struct.pack("<I", len(field)))
                out.write(field)


def read_metadata(path: str | Path) -> tuple[list[str], list[str]]:
    data = Path(path).read_bytes()
    magic, version, count = struct.unpack_from("<4sIq", data, 0)
    if magic != METADATA_MAGIC:
        raise ValueError("not a ZCVM metadata file")
    if version != METADATA_VERSION:
        raise ValueError(f"unsupported metadata version {version}")
    pos = 16
    ids, texts = [], []
    for _ in range(count):
        fields = []
        for _ in range(2):
            (length,) = struct.unpack_from("<I", data, pos)
            pos += 4
            fields.append(data[pos:pos + length].decode("utf-8"))
            pos += length
        ids.append(fields[0])
        texts.append(fields[1])
    return ids, texts


_LEX_HEADER = struct.Struct("<4sIqiqfff")


def write_lexical_index(path: str | Path, *, doc_count: int, vocab_size: int, offsets: np.ndarray,
                        posting_docs: np.ndarray, posting_weights: np.ndarray, k1: float, b: float,
                        average_doc_length: float) -> None:
    offsets = np.asarray(offsets, dtype=np.int64)
    docs = np.asarray(posting_docs, dtype=np.int32)
    weights = np.asarray(posting_weights, dtype=np.float32)
    if offsets.shape != (vocab_size + 1,) or offsets[0] != 0 or offsets[-1] != docs.size or docs.size != weights.size:
        raise ValueError("inconsistent CSR arrays")
    with open(path, "wb") as out:
        out.write(_LEX_HEADER.pack(LEXICAL_MAGIC, LEXICAL_VERSION, doc_count, vocab_size, docs.size, k1, b,
                                   average_doc_length))
        out.write(offsets.astype("<i8").tobytes())
        out.write(docs.astype("<i4").tobytes())
        out.write(weights.astype("<f4").tobytes())


def read_lexical_index(path: str | Path) -> dict:
    data = Path(path).read_bytes()
    magic, version, doc_count, vocab_size, nnz, k1, b, avgdl = _LEX_HEADER.unpack_from(data, 0)
    if magic != LEXICAL_MAGIC:
        raise ValueError("not a ZCVL lexical index")
    if version != LEXICAL_VERSION:
        raise ValueError(f"unsupported lexical index version {version}")
    pos = _LEX_HEADER.size
    offsets = np.frombuffer(data, dtype="<i8", count=vocab_size + 1, offset=pos).astype(np.int64)
    pos += 8 * (vocab_size + 1)
    docs = np.frombuffer(data, dtype="<i4", count=nnz, offset=pos).astype(np.int32)
    pos += 4 * nnz
    weights = np.frombuffer(data, dtype="<f4", count=nnz, offset=pos).astype(np.float32)
    return {"doc_count": doc_count, "vocab_size": vocab_size, "nnz": nnz, "k1": k1, "b": b,
            "average_doc_length": avgdl, "offsets": offsets, "posting_docs": docs, "posting_weights": weights}
