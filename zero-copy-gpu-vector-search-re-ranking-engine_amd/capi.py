"""ctypes binding of the C ABI in include/zcgvs_hip.h (lib/libzcgvs_hip.so).

Every call checks the returned status and raises: ValueError for ZCGVS_ERR_INVALID_ARGUMENT (the
reference's std::invalid_argument), RuntimeError for ZCGVS_ERR_RUNTIME / ZCGVS_ERR_HIP (its
std::runtime_error / CudaError). Loading fails loudly when the library has not been built; there
is no CPU fallback.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "lib" / "libzcgvs_hip.so"

OK, ERR_INVALID_ARGUMENT, ERR_RUNTIME, ERR_HIP, ERR_UNSUPPORTED = 0, 1, 2, 3, 4
COSINE, DOT, L2 = 0, 1, 2
F32, F16, I8, BINARY = 0, 1, 2, 3
INT8_REFERENCE, INT8_PER_VECTOR = 0, 1
SEARCH_MATERIALIZE = 1
SEARCH_UNSORTED_POSTINGS = 2
SEARCH_SORTED_POSTINGS = 4
SEARCH_FORCE_EXACT_PASS = 8
SEARCH_TEST_TINY_SEGMENTS = 16
SEARCH_TEST_HIGH_THRESHOLD = 32
SEARCH_TEST_TINY_RERUN = 64

_vp = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_sz = ctypes.c_size_t
_f32 = ctypes.c_float


class DeviceInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 256), ("arch", ctypes.c_char * 64), ("total_memory", _sz),
                ("compute_units", _i32), ("clock_khz", _i32), ("memory_clock_khz", _i32),
                ("memory_bus_width", _i32), ("l2_cache_bytes", _i32), ("major", _i32),
                ("minor", _i32), ("peak_bandwidth_gbs", ctypes.c_double)]


class StoreDesc(ctypes.Structure):
    _fields_ = [("data", _vp), ("doc_count", _i64), ("dim", _i32), ("dtype", _i32),
                ("scale", _f32), ("row_scales", _vp)]


class SearchDesc(ctypes.Structure):
    _fields_ = [("corpus", StoreDesc), ("rescore", StoreDesc), ("queries", _vp), ("batch", _i32),
                ("k", _i32), ("metric", _i32), ("int8_mode", _i32), ("mask", _vp),
                ("rescore_candidates", _i32), ("lex_offsets", _vp), ("lex_docs", _vp),
                ("lex_weights", _vp), ("lex_doc_count", _i64), ("lex_vocab_size", _i32), ("query_terms", _vp),
                ("lexical_stride", _i32), ("dense_weight", _f32), ("flags", _i32),
                ("lex_slice_table", _vp)]


# name -> (restype, argtypes)
_SIGNATURES = {
    "zcgvs_last_error": (ctypes.c_char_p, []),
    "zcgvs_version": (ctypes.c_char_p, []),
    "zcgvs_device_count": (_i32, [ctypes.POINTER(_i32)]),
    "zcgvs_set_device": (_i32, [_i32]),
    "zcgvs_get_device": (_i32, [ctypes.POINTER(_i32)]),
    "zcgvs_device_query": (_i32, [_i32, ctypes.POINTER(DeviceInfo)]),
    "zcgvs_device_synchronize": (_i32, []),
    "zcgvs_measure_hbm_bandwidth": (_i32, [_sz, _i32, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]),
    "zcgvs_malloc": (_i32, [ctypes.POINTER(_vp), _sz]),
    "zcgvs_free": (_i32, [_vp]),
    "zcgvs_host_alloc": (_i32, [ctypes.POINTER(_vp), _sz]),
    "zcgvs_host_free": (_i32, [_vp]),
    "zcgvs_memcpy_h2d": (_i32, [_vp, _vp, _sz, _vp]),
    "zcgvs_memcpy_d2h": (_i32, [_vp, _vp, _sz, _vp]),
    "zcgvs_memcpy_d2d": (_i32, [_vp, _vp, _sz, _vp]),
    "zcgvs_memset": (_i32, [_vp, _i32, _sz, _vp]),
    "zcgvs_fill_u32": (_i32, [_vp, ctypes.c_uint32, _sz, _vp]),
    "zcgvs_stream_create": (_i32, [ctypes.POINTER(_vp)]),
    "zcgvs_stream_destroy": (_i32, [_vp]),
    "zcgvs_stream_synchronize": (_i32, [_vp]),
    "zcgvs_event_create": (_i32, [ctypes.POINTER(_vp)]),
    "zcgvs_event_destroy": (_i32, [_vp]),
    "zcgvs_event_record": (_i32, [_vp, _vp]),
    "zcgvs_event_synchronize": (_i32, [_vp]),
    "zcgvs_event_elapsed_ms": (_i32, [ctypes.POINTER(_f32), _vp, _vp]),
    "zcgvs_graph_begin_capture": (_i32, [_vp]),
    "zcgvs_graph_end_capture": (_i32, [_vp, ctypes.POINTER(_vp)]),
    "zcgvs_graph_launch": (_i32, [_vp, _vp]),
    "zcgvs_graph_destroy": (_i32, [_vp]),
    "zcgvs_launch_similarity": (_i32, [_vp, _i32, _f32, _i32, _i32, _vp, _i32, _vp, _i32, _vp, _vp]),
    "zcgvs_launch_similarity_i8i8": (_i32, [_vp, _vp, _i32, _i32, _vp, _vp, _i32, _vp, _i32, _vp, _vp]),
    "zcgvs_similarity_query_tile": (_i32, []),
    "zcgvs_similarity_shared_bytes": (_sz, [_i32, _i32, _i32]),
    "zcgvs_topk_tile_size": (_i32, []),
    "zcgvs_topk_merge_tile": (_i32, []),
    "zcgvs_topk_max_k": (_i32, []),
    "zcgvs_topk_block_count": (_i32, [_i32]),
    "zcgvs_topk_scratch_elements": (_i32, [_i32, _i32]),
    "zcgvs_launch_topk": (_i32, [_vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "zcgvs_rescore_shared_bytes": (_sz, [_i32]),
    "zcgvs_launch_gather_rescore": (_i32, [_vp, _i32, _f32, _i32, _i32, _vp, _i32, _vp, _i32, _i32, _vp, _vp]),
    "zcgvs_launch_remap_indices": (_i32, [_vp, _vp, _i32, _i32, _i32, _vp, _vp]),
    "zcgvs_launch_bm25": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _vp, _vp]),
    "zcgvs_launch_bm25_batched": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp, _vp]),
    "zcgvs_lexical_slice_table_bytes": (_sz, [_i32, _i64]),
    "zcgvs_build_lexical_slice_table": (_i32, [_vp, _vp, _i32, _i64, _vp, _vp]),
    "zcgvs_launch_max_positive": (_i32, [_vp, _i32, _vp, _vp]),
    "zcgvs_launch_fuse_scores": (_i32, [_vp, _vp, _vp, _f32, _i32, _vp]),
    "zcgvs_launch_convert_f32_to_f16": (_i32, [_vp, _vp, _sz, _vp]),
    "zcgvs_launch_convert_f32_to_i8": (_i32, [_vp, _vp, _sz, _f32, _vp]),
    "zcgvs_launch_pack_binary": (_i32, [_vp, _vp, _i32, _i32, _vp]),
    "zcgvs_launch_quantize_rows_i8": (_i32, [_vp, _i32, _i32, _vp, _vp, _vp]),
    "zcgvs_search_workspace_bytes": (_sz, [ctypes.POINTER(SearchDesc)]),
    "zcgvs_search_topk": (_i32, [ctypes.POINTER(SearchDesc), _vp, _sz, _vp, _vp, _vp]),
    "zcgvs_search_topk_noalloc": (_i32, [ctypes.POINTER(SearchDesc), _vp, _vp, _vp]),
    "zcgvs_static_scratch_bytes": (_sz, []),
    "zcgvs_search_overflow_flags": (_i32, [ctypes.POINTER(SearchDesc), _vp, ctypes.POINTER(_vp)]),
    "zcgvs_search_sketch_state": (_i32, [ctypes.POINTER(SearchDesc), _vp, ctypes.POINTER(_vp), ctypes.POINTER(_i32),
                                         ctypes.POINTER(_i32), ctypes.POINTER(_i32), ctypes.POINTER(_vp),
                                         ctypes.POINTER(_vp)]),
    "zcgvs_search_topk_profiled": (_i32, [ctypes.POINTER(SearchDesc), _vp, _sz, _vp, _vp, _vp,
                                          ctypes.POINTER(_vp), _i32, ctypes.POINTER(_i32)]),
    "zcgvs_search_phase_rows": (_i32, [ctypes.POINTER(SearchDesc), ctypes.POINTER(_i64), _i32,
                                       ctypes.POINTER(_i32)]),
    "zcgvs_generate_normalized": (_i32, [_vp, _i64, _i32, _u64, _i64, _vp]),
}

_lib: ctypes.CDLL | None = None


def library() -> ctypes.CDLL:
    """The loaded HIP library; raises if it was never built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"zcgvs: {LIB_PATH} is missing; build it with `python build.py` (there is no CPU fallback)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def last_error() -> str:
    return library().zcgvs_last_error().decode()


def check(status: int) -> None:
    if status == OK:
        return
    message = last_error()
    if status == ERR_INVALID_ARGUMENT:
        raise ValueError(message)
    raise RuntimeError(message)


def call(name: str, *args) -> None:
    check(getattr(library(), name)(*args))


def ptr(x) -> int:
    """Device or host address of a DeviceArray / numpy array / int / None."""
    if x is None:
        return 0
    if isinstance(x, DeviceArray):
        return x.ptr
    if isinstance(x, np.ndarray):
        return x.ctypes.data
    return int(x)


class DeviceArray:
    """A device allocation with a numpy dtype and shape (RAII like include/zcgvs/core/device_buffer.hpp)."""

    def __init__(self, shape, dtype, zero=False):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        address = _vp()
        call("zcgvs_malloc", ctypes.byref(address), max(self.nbytes, 1))
        self.ptr = int(address.value or 0)
        if zero:
            call("zcgvs_memset", self.ptr, 0, self.nbytes, None)
            synchronize()

    @classmethod
    def from_host(cls, array: np.ndarray) -> "DeviceArray":
        array = np.ascontiguousarray(array)
        out = cls(array.shape, array.dtype)
        call("zcgvs_memcpy_h2d", out.ptr, array.ctypes.data, array.nbytes, None)
        synchronize()
        return out

    def to_host(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        call("zcgvs_memcpy_d2h", out.ctypes.data, self.ptr, self.nbytes, None)
        synchronize()
        return out

    def free(self) -> None:
        if self.ptr:
            call("zcgvs_free", self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            if self.ptr and _lib is not None:
                _lib.zcgvs_free(self.ptr)
                self.ptr = 0
        except Exception:  # interpreter shutdown
            pass


def synchronize() -> None:
    call("zcgvs_device_synchronize")


def device_count() -> int:
    count = _i32(0)
    status = library().zcgvs_device_count(ctypes.byref(count))
    return count.value if status == OK else 0


def device_info(device: int = 0) -> DeviceInfo:
    info = DeviceInfo()
    call("zcgvs_device_query", device, ctypes.byref(info))
    return info


def measure_hbm_bandwidth(nbytes: int = 4 << 30, iterations: int = 5) -> tuple[float, float]:
    """(read GB/s, copy GB/s) of the current device, measured by streaming kernels."""
    read, copy = ctypes.c_double(0.0), ctypes.c_double(0.0)
    call("zcgvs_measure_hbm_bandwidth", nbytes, iterations, ctypes.byref(read), ctypes.byref(copy))
    return read.value, copy.value


class Stream:
    def __init__(self):
        handle = _vp()
        call("zcgvs_stream_create", ctypes.byref(handle))
        self.handle = handle.value

    def synchronize(self) -> None:
        call("zcgvs_stream_synchronize", self.handle)

    def __del__(self):
        try:
            if self.handle and _lib is not None:
                _lib.zcgvs_stream_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


class Event:
    def __init__(self):
        handle = _vp()
        call("zcgvs_event_create", ctypes.byref(handle))
        self.handle = handle.value

    def record(self, stream=None) -> None:
        call("zcgvs_event_record", self.handle, getattr(stream, "handle", stream))

    def elapsed_ms(self, end: "Event") -> float:
        out = _f32(0.0)
        call("zcgvs_event_synchronize", end.handle)
        call("zcgvs_event_elapsed_ms", ctypes.byref(out), self.handle, end.handle)
        return float(out.value)

    def __del__(self):
        try:
            if self.handle and _lib is not None:
                _lib.zcgvs_event_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


class Graph:
    """The work `record()` enqueues on `stream`, captured once (zcgvs_graph_begin_capture /
    end_capture) and replayed with launch(); the reference's Searcher graph cache
    (src/search/searcher.cpp:287-342) does the same for a repeated query shape."""

    def __init__(self, stream: Stream, record):
        call("zcgvs_graph_begin_capture", stream.handle)
        handle = _vp()
        try:
            record()
        finally:
            # the capture must end even when recording failed; that error is the one raised
            status = library().zcgvs_graph_end_capture(stream.handle, ctypes.byref(handle))
        check(status)
        self.handle = handle.value

    def launch(self, stream: Stream) -> None:
        call("zcgvs_graph_launch", self.handle, stream.handle)

    def __del__(self):
        try:
            if getattr(self, "handle", None) and _lib is not None:
                _lib.zcgvs_graph_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


# ---- launcher wrappers (device pointers in, status checked) ---------------------------------

def launch_similarity(corpus, dtype, scale, n, dim, queries, batch, mask, metric, scores, stream=None):
    call("zcgvs_launch_similarity", ptr(corpus), dtype, scale, n, dim, ptr(queries), batch, ptr(mask),
         metric, ptr(scores), getattr(stream, "handle", stream))


def launch_similarity_i8i8(corpus, row_scales, n, dim, queries, query_scales, batch, mask, metric,
                           scores, stream=None):
    call("zcgvs_launch_similarity_i8i8", ptr(corpus), ptr(row_scales), n, dim, ptr(queries),
         ptr(query_scales), batch, ptr(mask), metric, ptr(scores), getattr(stream, "handle", stream))


def topk_scratch_elements(n, k) -> int:
    return int(library().zcgvs_topk_scratch_elements(n, k))


def launch_topk(scores, n, k, batch, out_idx, out_val, sa, ia, sb, ib, stream=None):
    call("zcgvs_launch_topk", ptr(scores), n, k, batch, ptr(out_idx), ptr(out_val), ptr(sa), ptr(ia),
         ptr(sb), ptr(ib), getattr(stream, "handle", stream))


def topk(scores: DeviceArray, k: int, stream=None):
    """Convenience: top-k of a device [B, N] float32 matrix -> host (idx, val)."""
    batch, n = scores.shape
    elements = topk_scratch_elements(n, k)
    scratch = [DeviceArray((batch, elements), np.float32), DeviceArray((batch, elements), np.int32),
               DeviceArray((batch, elements), np.float32), DeviceArray((batch, elements), np.int32)]
    idx = DeviceArray((batch, k), np.int32)
    val = DeviceArray((batch, k), np.float32)
    launch_topk(scores, n, k, batch, idx, val, *scratch, stream=stream)
    synchronize()
    return idx.to_host(), val.to_host()


def launch_gather_rescore(corpus, dtype, scale, n, dim, queries, batch, candidates, count, metric,
                          values, stream=None):
    call("zcgvs_launch_gather_rescore", ptr(corpus), dtype, scale, n, dim, ptr(queries), batch,
         ptr(candidates), count, metric, ptr(values), getattr(stream, "handle", stream))


def launch_remap_indices(candidates, local, count, k, batch, out, stream=None):
    call("zcgvs_launch_remap_indices", ptr(candidates), ptr(local), count, k, batch, ptr(out),
         getattr(stream, "handle", stream))


def launch_bm25(offsets, docs, weights, terms, term_count, n, scores, stream=None):
    call("zcgvs_launch_bm25", ptr(offsets), ptr(docs), ptr(weights), ptr(terms), term_count, n,
         ptr(scores), getattr(stream, "handle", stream))


def launch_bm25_batched(offsets, docs, weights, terms, stride, batch, n, scores, stream=None):
    call("zcgvs_launch_bm25_batched", ptr(offsets), ptr(docs), ptr(weights), ptr(terms), stride, batch,
         n, ptr(scores), getattr(stream, "handle", stream))


def lexical_slice_table_bytes(vocab_size, doc_count) -> int:
    """Bytes of the slice table of an index of `vocab_size` terms over `doc_count` documents
    (0 for an empty index or more than 2^31 - 1 documents)."""
    return int(library().zcgvs_lexical_slice_table_bytes(vocab_size, doc_count))


def build_lexical_slice_table(offsets, docs, vocab_size, doc_count, table, stream=None):
    """Fills `table` (lexical_slice_table_bytes of device memory, uint32) with, for every term
    and 4096-document boundary, the number of the term's postings below it (sorted postings)."""
    call("zcgvs_build_lexical_slice_table", ptr(offsets), ptr(docs), vocab_size, doc_count, ptr(table),
         getattr(stream, "handle", stream))


def launch_max_positive(values, count, out, stream=None):
    call("zcgvs_launch_max_positive", ptr(values), count, ptr(out), getattr(stream, "handle", stream))


def launch_fuse_scores(dense, lexical, lexical_max, weight, count, stream=None):
    call("zcgvs_launch_fuse_scores", ptr(dense), ptr(lexical), ptr(lexical_max), weight, count,
         getattr(stream, "handle", stream))


def launch_convert_f32_to_f16(src, dst, count, stream=None):
    call("zcgvs_launch_convert_f32_to_f16", ptr(src), ptr(dst), count, getattr(stream, "handle", stream))


def launch_convert_f32_to_i8(src, dst, count, scale, stream=None):
    call("zcgvs_launch_convert_f32_to_i8", ptr(src), ptr(dst), count, scale, getattr(stream, "handle", stream))


def launch_pack_binary(src, dst, rows, dim, stream=None):
    call("zcgvs_launch_pack_binary", ptr(src), ptr(dst), rows, dim, getattr(stream, "handle", stream))


def launch_quantize_rows_i8(src, rows, dim, dst, scales, stream=None):
    call("zcgvs_launch_quantize_rows_i8", ptr(src), rows, dim, ptr(dst), ptr(scales),
         getattr(stream, "handle", stream))


def generate_normalized(out, rows, dim, seed, row_offset=0, stream=None):
    call("zcgvs_generate_normalized", ptr(out), rows, dim, seed, row_offset, getattr(stream, "handle", stream))


# ---- fused search --------------------------------------------------------------------------

def _keep_alive(desc, *owners):
    """Descriptors hold raw device addresses; keep the Python objects that own that memory alive
    for as long as the descriptor lives, so a temporary DeviceArray passed to a descriptor
    builder is not freed (hipFree) while a kernel still reads it."""
    keep = getattr(desc, "_owners", [])
    keep.extend(o for o in owners if o is not None and not isinstance(o, int))
    desc._owners = keep
    return desc


def store_desc(data=None, doc_count=0, dim=0, dtype=F32, scale=1.0, row_scales=None) -> StoreDesc:
    return _keep_alive(StoreDesc(ptr(data), doc_count, dim, dtype, scale, ptr(row_scales)),
                       data, row_scales)


def search_desc(corpus: StoreDesc, queries, batch, k, metric=COSINE, *, int8_mode=INT8_REFERENCE,
                mask=None, rescore: StoreDesc | None = None, rescore_candidates=0, lex_offsets=None,
                lex_docs=None, lex_weights=None, lex_doc_count=0, lex_vocab_size=0, query_terms=None,
                lexical_stride=0, dense_weight=1.0, flags=0, lex_slice_table=None) -> SearchDesc:
    desc = SearchDesc(corpus, rescore if rescore is not None else StoreDesc(), ptr(queries), batch, k,
                      metric, int8_mode, ptr(mask), rescore_candidates, ptr(lex_offsets), ptr(lex_docs),
                      ptr(lex_weights), lex_doc_count, lex_vocab_size, ptr(query_terms), lexical_stride,
                      dense_weight, flags, ptr(lex_slice_table))
    # the nested StoreDesc fields are copied by value: carry their owners over as well
    return _keep_alive(desc, *getattr(corpus, "_owners", []),
                       *(getattr(rescore, "_owners", []) if rescore is not None else []),
                       queries, mask, lex_offsets, lex_docs, lex_weights, query_terms, lex_slice_table)


def search_workspace_bytes(desc: SearchDesc) -> int:
    size = int(library().zcgvs_search_workspace_bytes(ctypes.byref(desc)))
    if size == 0:
        message = last_error()
        if message:
            if "exceeds the supported document count" in message:
                raise RuntimeError(message)
            raise ValueError(message)
    return size


def search_topk(desc: SearchDesc, workspace, workspace_bytes, out_idx, out_val, stream=None) -> None:
    call("zcgvs_search_topk", ctypes.byref(desc), ptr(workspace), workspace_bytes, ptr(out_idx),
         ptr(out_val), getattr(stream, "handle", stream))


def search_topk_profiled(desc: SearchDesc, workspace, workspace_bytes, out_idx, out_val, stream,
                         events: list, max_phases: int) -> int:
    """zcgvs_search_topk recording events[2p], events[2p+1] around the scan of phase p."""
    handles = (_vp * (2 * max_phases))(*[e.handle for e in events])
    phases = _i32(0)
    call("zcgvs_search_topk_profiled", ctypes.byref(desc), ptr(workspace), workspace_bytes, ptr(out_idx),
         ptr(out_val), getattr(stream, "handle", stream), handles, max_phases, ctypes.byref(phases))
    return phases.value


def search_phase_rows(desc: SearchDesc, max_phases: int = 16) -> list[int]:
    """Corpus rows each scan phase visits (empty when the pipeline materializes scores)."""
    rows = (_i64 * max_phases)()
    phases = _i32(0)
    call("zcgvs_search_phase_rows", ctypes.byref(desc), rows, max_phases, ctypes.byref(phases))
    return [int(rows[p]) for p in range(min(phases.value, max_phases))]


def search_overflow_flags(desc: SearchDesc, workspace) -> int:
    address = _vp()
    call("zcgvs_search_overflow_flags", ctypes.byref(desc), ptr(workspace), ctypes.byref(address))
    return int(address.value or 0)


def search_sketch_state(desc: SearchDesc, workspace) -> dict | None:
    """A completed sketch-planned search's slot scores [slots, batch] and thresholds (host copies),
    or None when the search is not sketch-planned."""
    scores, tau, tau_safe = _vp(), _vp(), _vp()
    slots, rank, width = _i32(0), _i32(0), _i32(0)
    call("zcgvs_search_sketch_state", ctypes.byref(desc), ptr(workspace), ctypes.byref(scores), ctypes.byref(slots),
         ctypes.byref(rank), ctypes.byref(width), ctypes.byref(tau), ctypes.byref(tau_safe))
    if slots.value == 0:
        return None
    out = dict(slots=np.empty((slots.value, desc.batch), dtype=np.float32), rank=rank.value, width=width.value,
               tau=np.empty(desc.batch, dtype=np.uint64), tau_safe=np.empty(desc.batch, dtype=np.uint64))
    synchronize()
    for name, address in (("slots", scores), ("tau", tau), ("tau_safe", tau_safe)):
        call("zcgvs_memcpy_d2h", out[name].ctypes.data, address.value, out[name].nbytes, None)
    synchronize()
    return out


def search(desc: SearchDesc, stream=None):
    """Convenience: run the fused search with a fresh workspace -> host (idx, val, overflow)."""
    size = search_workspace_bytes(desc)
    workspace = DeviceArray(size, np.uint8)
    idx = DeviceArray((desc.batch, desc.k), np.int32)
    val = DeviceArray((desc.batch, desc.k), np.float32)
    search_topk(desc, workspace, size, idx, val, stream)
    synchronize()
    flags = np.empty(desc.batch, dtype=np.uint32)
    call("zcgvs_memcpy_d2h", flags.ctypes.data, search_overflow_flags(desc, workspace), flags.nbytes, None)
    synchronize()
    return idx.to_host(), val.to_host(), flags
