"""CPU oracle of the zero-copy search hot path - TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package,
and only to check results (or as the timed CPU baseline); the product path never calls it.

`oracle.c` (built to _build/liboracle.so by the Makefile) restates the reference's CPU semantics
function by function; `ref` gives the reference's own tests/cpp/cpu_reference.hpp compiled from
the reference checkout into _ref/libcpuref.so, when that was available at build time.
Everything here takes and returns numpy arrays.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"
REF_PATH = HERE / "_ref" / "libcpuref.so"

COSINE, DOT, L2 = 0, 1, 2
FLT_MAX = float(np.finfo(np.float32).max)

_lib = None
_ref = None


def _ptr(array: np.ndarray | None) -> ctypes.c_void_p:
    if array is None:
        return ctypes.c_void_p(0)
    return ctypes.c_void_p(array.ctypes.data)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run `make -C oracle`)")
        _lib = ctypes.CDLL(str(LIB_PATH))
        _lib.zo_hamming.restype = ctypes.c_int
        _lib.zo_max_positive.restype = ctypes.c_float
        _lib.zo_threads.restype = ctypes.c_int
        _lib.zo_bm25_weight.restype = ctypes.c_float
        _lib.zo_bm25_weight.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int32,
                                        ctypes.c_double, ctypes.c_double, ctypes.c_double,
                                        ctypes.c_double]
    return _lib


def ref() -> ctypes.CDLL | None:
    """The reference's own CPU path, or None when it was not built."""
    global _ref
    if _ref is None and REF_PATH.exists():
        _ref = ctypes.CDLL(str(REF_PATH))
        _ref.ref_hamming.restype = ctypes.c_int
    return _ref


def _c(array, dtype) -> np.ndarray:
    return np.ascontiguousarray(array, dtype=dtype)


# ---- scores ------------------------------------------------------------------------------

def scores_f32(corpus, queries, metric=COSINE, mask=None) -> np.ndarray:
    """[B, N] sequential float32 scores of a float32 (or decoded) corpus."""
    corpus = _c(corpus, np.float32)
    queries = _c(np.atleast_2d(queries), np.float32)
    n, dim = corpus.shape
    out = np.empty((queries.shape[0], n), dtype=np.float32)
    mask = None if mask is None else _c(mask, np.uint8)
    lib().zo_scores_f32(_ptr(corpus), ctypes.c_int64(n), ctypes.c_int(dim), _ptr(queries),
                        ctypes.c_int(queries.shape[0]), _ptr(mask), ctypes.c_int(metric), _ptr(out))
    return out


def scores_i8i8(corpus, row_scales, queries, query_scales, mask=None) -> np.ndarray:
    corpus = _c(corpus, np.int8)
    queries = _c(np.atleast_2d(queries), np.int8)
    row_scales = _c(row_scales, np.float32)
    query_scales = _c(query_scales, np.float32)
    n, dim = corpus.shape
    out = np.empty((queries.shape[0], n), dtype=np.float32)
    mask = None if mask is None else _c(mask, np.uint8)
    lib().zo_scores_i8i8(_ptr(corpus), _ptr(row_scales), ctypes.c_int64(n), ctypes.c_int(dim),
                         _ptr(queries), _ptr(query_scales), ctypes.c_int(queries.shape[0]),
                         _ptr(mask), _ptr(out))
    return out


def scores_hamming(corpus_words, query_words, dim, mask=None) -> np.ndarray:
    corpus_words = _c(corpus_words, np.uint32)
    query_words = _c(np.atleast_2d(query_words), np.uint32)
    n = corpus_words.shape[0]
    out = np.empty((query_words.shape[0], n), dtype=np.float32)
    mask = None if mask is None else _c(mask, np.uint8)
    lib().zo_scores_hamming(_ptr(corpus_words), ctypes.c_int64(n), ctypes.c_int(dim),
                            _ptr(query_words), ctypes.c_int(query_words.shape[0]), _ptr(mask),
                            _ptr(out))
    return out


def hamming(a, b) -> int:
    a = _c(a, np.uint32)
    b = _c(b, np.uint32)
    return int(lib().zo_hamming(_ptr(a), _ptr(b), ctypes.c_int(a.size)))


# ---- conversions -------------------------------------------------------------------------

def f32_to_f16(values) -> np.ndarray:
    values = _c(values, np.float32)
    out = np.empty(values.shape, dtype=np.uint16)
    lib().zo_f32_to_f16(_ptr(values), ctypes.c_int64(values.size), _ptr(out))
    return out.view(np.float16)


def f16_to_f32(values) -> np.ndarray:
    values = _c(values, np.float16).view(np.uint16)
    out = np.empty(values.shape, dtype=np.float32)
    lib().zo_f16_to_f32(_ptr(values), ctypes.c_int64(values.size), _ptr(out))
    return out


def quantize_i8(values, scale) -> np.ndarray:
    values = _c(values, np.float32)
    out = np.empty(values.shape, dtype=np.int8)
    lib().zo_quantize_i8(_ptr(values), ctypes.c_int64(values.size), ctypes.c_float(scale), _ptr(out))
    return out


def dequantize_i8(codes, scale) -> np.ndarray:
    codes = _c(codes, np.int8)
    out = np.empty(codes.shape, dtype=np.float32)
    lib().zo_dequantize_i8(_ptr(codes), ctypes.c_int64(codes.size), ctypes.c_float(scale), _ptr(out))
    return out


def quantize_dequantize_i8(values, scale) -> np.ndarray:
    values = _c(values, np.float32)
    out = np.empty(values.shape, dtype=np.float32)
    lib().zo_quantize_dequantize_i8(_ptr(values), ctypes.c_int64(values.size), ctypes.c_float(scale), _ptr(out))
    return out


def quantize_rows_i8(values) -> tuple[np.ndarray, np.ndarray]:
    values = _c(np.atleast_2d(values), np.float32)
    rows, dim = values.shape
    codes = np.empty((rows, dim), dtype=np.int8)
    scales = np.empty(rows, dtype=np.float32)
    lib().zo_quantize_rows_i8(_ptr(values), ctypes.c_int64(rows), ctypes.c_int(dim), _ptr(codes), _ptr(scales))
    return codes, scales


def pack_binary(values) -> np.ndarray:
    values = _c(np.atleast_2d(values), np.float32)
    rows, dim = values.shape
    out = np.empty((rows, (dim + 31) // 32), dtype=np.uint32)
    lib().zo_pack_binary(_ptr(values), ctypes.c_int64(rows), ctypes.c_int(dim), _ptr(out))
    return out


def l2_normalize(values) -> np.ndarray:
    values = _c(np.atleast_2d(values), np.float32).copy()
    lib().zo_l2_normalize(_ptr(values), ctypes.c_int64(values.shape[0]), ctypes.c_int(values.shape[1]))
    return values


# ---- selection ---------------------------------------------------------------------------

def topk(scores, k) -> tuple[np.ndarray, np.ndarray]:
    """(indices [B, k] int32, scores [B, k] float32), score desc then index asc."""
    scores = _c(np.atleast_2d(scores), np.float32)
    batch, n = scores.shape
    idx = np.empty((batch, k), dtype=np.int32)
    val = np.empty((batch, k), dtype=np.float32)
    lib().zo_topk(_ptr(scores), ctypes.c_int64(n), ctypes.c_int(batch), ctypes.c_int(k), _ptr(idx), _ptr(val))
    return idx, val


# ---- rescore / lexical -------------------------------------------------------------------

def rescore(store, queries, candidates, metric=COSINE) -> np.ndarray:
    store = _c(store, np.float32)
    queries = _c(np.atleast_2d(queries), np.float32)
    candidates = _c(np.atleast_2d(candidates), np.int32)
    n, dim = store.shape
    batch, count = candidates.shape
    out = np.empty((batch, count), dtype=np.float32)
    lib().zo_rescore(_ptr(store), ctypes.c_int64(n), ctypes.c_int(dim), _ptr(queries), ctypes.c_int(batch),
                     _ptr(candidates), ctypes.c_int(count), ctypes.c_int(metric), _ptr(out))
    return out


def remap(candidates, local) -> np.ndarray:
    candidates = _c(np.atleast_2d(candidates), np.int32)
    local = _c(np.atleast_2d(local), np.int32)
    batch, count = candidates.shape
    k = local.shape[1]
    out = np.empty((batch, k), dtype=np.int32)
    lib().zo_remap(_ptr(candidates), _ptr(local), ctypes.c_int(count), ctypes.c_int(k), ctypes.c_int(batch), _ptr(out))
    return out


def bm25(offsets, docs, weights, terms, n) -> np.ndarray:
    offsets = _c(offsets, np.int64)
    docs = _c(docs, np.int32)
    weights = _c(weights, np.float32)
    terms = _c(terms, np.int32)
    out = np.empty(n, dtype=np.float32)
    lib().zo_bm25(_ptr(offsets), _ptr(docs), _ptr(weights), _ptr(terms), ctypes.c_int(terms.size),
                  ctypes.c_int64(n), _ptr(out))
    return out


def max_positive(values) -> float:
    values = _c(values, np.float32)
    return float(lib().zo_max_positive(_ptr(values), ctypes.c_int64(values.size)))


def fuse(dense, lexical, lexical_max, weight) -> np.ndarray:
    dense = _c(dense, np.float32).copy()
    lexical = _c(lexical, np.float32)
    lib().zo_fuse(_ptr(dense), _ptr(lexical), ctypes.c_float(lexical_max), ctypes.c_float(weight),
                  ctypes.c_int64(dense.size))
    return dense


def bm25_weight(doc_count, df, tf, length, average_length, k1=1.2, b=0.75) -> float:
    return float(lib().zo_bm25_weight(doc_count, df, tf, float(length), float(average_length),
                                      float(k1), float(b)))


def threads() -> int:
    """OpenMP threads the parallel score loops use."""
    return int(lib().zo_threads())


def set_threads(count: int) -> None:
    """Thread count of the parallel loops (every result is independent of it)."""
    lib().zo_set_threads(ctypes.c_int(count))
