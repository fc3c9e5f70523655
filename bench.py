#!/usr/bin/env python3
"""Benchmark of the zero-copy search hot path on one MI355X.

A step is one fused search of a resident query batch against a resident corpus (the device
pipeline of src/search/searcher.cpp:209-285: scan, selection, optional rescore). K steps run back
to back on one stream, timed by the host clock with the device synchronized on both sides; the
per-step latency (p50) and the scan launches' durations come from HIP events in K untimed
repeats each. Inputs are synthetic (seeded, generated on the device) and in HBM before timing
starts; only [batch, k] ids and scores are produced.

Default workload (the per-vector int8 configuration): 10,000,000 x 768 int8 rows, per-row scale
max|x|/127, 256 queries quantized the same way on the device, k = 100, int8 MFMA contraction.
Other workloads: --workload NAME (see WORKLOADS).

Prints one JSON line: queries/s over the timed steps, p50 step latency, the scan kernel's
roofline (algorithmic bytes / scan time, from events around the scan launches), and the CPU
oracle timed on a bounded sample of the same queries on this host (with a full-size parity
check of the sampled queries against the GPU result). The default run also measures, under
"secondary", the other benchmark configurations (float32 5,183 x 384; float32 and float16
1M x 384 at batch 1 and 64; per-vector int8 10M x 768 at batch 1; binary 50M x 1024 with a
float16 rescore; hybrid BM25 + float16 1M x 384), each with its step time, roofline fraction and
a sampled parity check, and under "reference_tables" the shapes apps/bench_kernels.cu:151-273
times: the storage-type scan (the similarity launcher, 1M x 384, one query), top-k selection over
1M scores at k = 10, 100, 1000, and the float16 1M x 384 k = 100 pipeline at batch 1, 8, 32 with
direct launches and with graph replay. --no-secondary skips both.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from __graft_entry__ import load_package  # noqa: E402

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, published
INT8_MFMA_PEAK_TOPS = 5000.0   # MI355X dense int8 MFMA, published
FP4_MFMA_PEAK_TOPS = 10100.0   # MI355X dense fp4 MFMA, published (the binary scans' operands)
CORPUS_SEED = 1234
QUERY_SEED = 4321

WORKLOADS = {
    "int8-10m": dict(kind="i8i8", n=10_000_000, dim=768, batch=256, k=100,
                     name="per-vector int8 10M x 768, batch 256, k=100"),
    "int8-10m-b1": dict(kind="i8i8", n=10_000_000, dim=768, batch=1, k=100,
                        name="per-vector int8 10M x 768, batch 1, k=100"),
    "int8-10m-sorted": dict(kind="i8i8", n=10_000_000, dim=768, batch=256, k=100, sort_rows=True,
                            name="per-vector int8 10M x 768 with rows sorted by their first coordinate, "
                                 "batch 256, k=100"),
    "int8-10m-hot": dict(kind="i8i8", n=10_000_000, dim=768, batch=256, k=100, hot_queries=16, hot_blocks=4,
                         name="per-vector int8 10M x 768 with 256 near-copies of each of 16 queries crowded "
                              "into one workgroup's blocks, batch 256, k=100"),
    "f32-1m-b1": dict(kind="f32", n=1_000_000, dim=384, batch=1, k=10,
                      name="float32 1M x 384, batch 1, k=10"),
    "f16-1m-b1": dict(kind="f16", n=1_000_000, dim=384, batch=1, k=10,
                      name="float16 1M x 384, batch 1, k=10"),
    "f32-1m-b64": dict(kind="f32", n=1_000_000, dim=384, batch=64, k=10,
                       name="float32 1M x 384, batch 64, k=10"),
    "f16-1m-b64": dict(kind="f16", n=1_000_000, dim=384, batch=64, k=10,
                       name="float16 1M x 384, batch 64, k=10"),
    "binary-50m": dict(kind="binary", n=50_000_000, dim=1024, batch=32, k=10, candidates=1000,
                       name="binary 50M x 1024 + float16 rescore of 1000, batch 32, k=10"),
    "binary-50m-b1": dict(kind="binary", n=50_000_000, dim=1024, batch=1, k=10, candidates=1000,
                          name="binary 50M x 1024 + float16 rescore of 1000, batch 1, k=10"),
    "binary-50m-b128": dict(kind="binary", n=50_000_000, dim=1024, batch=128, k=10, candidates=1000,
                            name="binary 50M x 1024 + float16 rescore of 1000, batch 128, k=10"),
    "hybrid-1m": dict(kind="hybrid", n=1_000_000, dim=384, batch=16, k=10, vocab=30_000, terms=8,
                      dense_weight=0.5,
                      name="hybrid BM25 (V=30,000, 8-term queries) + float16 1M x 384 cosine, batch 16, k=10"),
    "cpu-ref": dict(kind="f32", n=5183, dim=384, batch=1, k=10,
                    name="float32 5,183 x 384, batch 1, k=10"),
}
LEXICAL_SEED = 7
TERMS_SEED = 11
HOT_SEED = 13


def log(*args):
    print("[bench]", *args, file=sys.stderr, flush=True)


def build_inputs(capi, w):
    """Corpus, queries and search descriptor on the device."""
    n, dim, batch = w["n"], w["dim"], w["batch"]
    kind = w["kind"]
    keep = {}
    chunk = max(1, min(n, (2 << 30) // (dim * 4)))
    stage = capi.DeviceArray((chunk, dim), np.float32)
    if kind == "i8i8":
        corpus = capi.DeviceArray((n, dim), np.int8)
        scales = capi.DeviceArray(n, np.float32)
        keep["scales"] = scales
    elif kind == "f32":
        corpus = capi.DeviceArray((n, dim), np.float32)
    elif kind in ("f16", "hybrid"):
        corpus = capi.DeviceArray((n, dim), np.float16)
    else:
        corpus = capi.DeviceArray((n, (dim + 31) // 32), np.uint32)
        rescore = capi.DeviceArray((n, dim), np.float16)
        keep["rescore"] = rescore
    for start in range(0, n, chunk):
        rows = min(chunk, n - start)
        capi.generate_normalized(stage, rows, dim, CORPUS_SEED, start)
        if kind == "i8i8":
            capi.launch_quantize_rows_i8(stage, rows, dim, corpus.ptr + start * dim, scales.ptr + start * 4)
        elif kind == "f32":
            capi.call("zcgvs_memcpy_d2d", corpus.ptr + start * dim * 4, stage.ptr, rows * dim * 4, None)
        elif kind in ("f16", "hybrid"):
            capi.launch_convert_f32_to_f16(stage, corpus.ptr + start * dim * 2, rows * dim)
        else:
            words = (dim + 31) // 32
            capi.launch_pack_binary(stage, corpus.ptr + start * words * 4, rows, dim)
            capi.launch_convert_f32_to_f16(stage, rescore.ptr + start * dim * 2, rows * dim)
        capi.synchronize()
    stage.free()
    if w.get("sort_rows"):
        # a clustered corpus: rows in ascending order of their first coordinate, so a query's
        # best rows crowd into one end of the corpus instead of being spread over it
        log("sorting the corpus rows by their first coordinate")
        codes = corpus.to_host()
        order = np.argsort(codes[:, 0], kind="stable")
        codes = np.ascontiguousarray(codes[order])
        capi.call("zcgvs_memcpy_h2d", corpus.ptr, codes.ctypes.data, codes.nbytes, None)
        row_scales = np.ascontiguousarray(keep["scales"].to_host()[order])
        capi.call("zcgvs_memcpy_h2d", keep["scales"].ptr, row_scales.ctypes.data, row_scales.nbytes, None)
        capi.synchronize()
        del codes, row_scales, order
    queries = capi.DeviceArray((batch, dim), np.float32)
    capi.generate_normalized(queries, batch, dim, QUERY_SEED, 0)
    capi.synchronize()
    if w.get("hot_queries"):
        # A corpus whose best rows crowd together: for each of the first hot_queries queries,
        # hot_blocks 64-row blocks of near-copies of it (the query plus 2% noise per dimension, normalized),
        # placed at blocks 1 + cu * m, so one workgroup of a scan with one workgroup per CU visits
        # them all (and the sketch's every-32nd-block sample none): those queries' candidates
        # overflow that workgroup's buffers and take the exact fallback.
        cus = capi.device_info(0).compute_units
        host_q = queries.to_host()
        rng = np.random.default_rng(HOT_SEED)
        hot = capi.DeviceArray((64, dim), np.float32)
        block = 0
        for b in range(w["hot_queries"]):
            for _ in range(w["hot_blocks"]):
                rows = host_q[b] + np.float32(0.02) * rng.standard_normal((64, dim)).astype(np.float32)
                rows /= np.linalg.norm(rows, axis=1, keepdims=True)
                rows = np.ascontiguousarray(rows, dtype=np.float32)
                capi.call("zcgvs_memcpy_h2d", hot.ptr, rows.ctypes.data, rows.nbytes, None)
                first = (1 + cus * block) * 64
                capi.launch_quantize_rows_i8(hot, 64, dim, corpus.ptr + first * dim,
                                             keep["scales"].ptr + first * 4)
                capi.synchronize()
                block += 1
        hot.free()
        keep["hot_rows"] = [(1 + cus * m) * 64 for m in range(block)]
    dtype = {"i8i8": capi.I8, "f32": capi.F32, "f16": capi.F16, "hybrid": capi.F16, "binary": capi.BINARY}[kind]
    store = capi.store_desc(corpus, n, dim, dtype, 1.0, keep.get("scales"))
    extra = {}
    if kind == "i8i8":
        extra["int8_mode"] = capi.INT8_PER_VECTOR
    if kind == "binary":
        extra["rescore"] = capi.store_desc(keep["rescore"], n, dim, capi.F16)
        extra["rescore_candidates"] = w["candidates"]
    if kind == "hybrid":
        from zcgvs_amd.zcgvs_tools import lexical
        log(f"building the synthetic BM25 index ({n:,} documents, vocabulary {w['vocab']:,})")
        index = lexical.synthetic_index(n, w["vocab"], seed=LEXICAL_SEED)
        terms = lexical.synthetic_queries(batch, w["terms"], w["vocab"], seed=TERMS_SEED)
        keep["lexical"] = {name: capi.DeviceArray.from_host(index[name])
                           for name in ("offsets", "posting_docs", "posting_weights")}
        keep["terms"] = capi.DeviceArray.from_host(terms)
        # the index's slice table (built once with the index, outside every timed region)
        table_bytes = capi.lexical_slice_table_bytes(w["vocab"], n)
        keep["slice_table"] = capi.DeviceArray(table_bytes // 4, np.uint32)
        capi.build_lexical_slice_table(keep["lexical"]["offsets"], keep["lexical"]["posting_docs"], w["vocab"], n,
                                       keep["slice_table"])
        capi.synchronize()
        keep["postings"] = int(index["offsets"][-1])
        keep["index"] = index
        keep["terms_host"] = terms
        extra.update(lex_offsets=keep["lexical"]["offsets"], lex_docs=keep["lexical"]["posting_docs"],
                     lex_weights=keep["lexical"]["posting_weights"], lex_doc_count=n,
                     lex_vocab_size=w["vocab"], query_terms=keep["terms"], lexical_stride=w["terms"],
                     dense_weight=w["dense_weight"], flags=capi.SEARCH_SORTED_POSTINGS,
                     lex_slice_table=keep["slice_table"])
    desc = capi.search_desc(store, queries, batch, w["k"], capi.COSINE, **extra)
    return desc, corpus, queries, keep


def row_bytes(w):
    """Algorithmic HBM bytes per corpus row a scan reads (row + its per-row scale). A hybrid scan
    also reads each row's [batch] lexical scores, an intermediate of this design that the
    reference's order of stages does not have; that is overhead, not counted here."""
    dim = w["dim"]
    return {"i8i8": dim + 4, "f32": dim * 4, "f16": dim * 2, "hybrid": dim * 2,
            "binary": (dim + 31) // 32 * 4}[w["kind"]]


def lexical_bytes(keep):
    """Algorithmic bytes of the batch's BM25 stage: 8 B (doc id + weight) per posting of every
    query's terms, plus the two 8-byte offsets of each term (the stage's HBM-roofline numerator)."""
    terms = keep["terms_host"]
    offsets = keep["index"]["offsets"]
    valid = terms >= 0
    t = np.where(valid, terms, 0)
    df = np.where(valid, offsets[t + 1] - offsets[t], 0)
    return int(df.sum()) * 8 + int(valid.sum()) * 16


def query_bytes(w):
    """Bytes of the (device-prepared) queries one scan launch reads."""
    dim, batch = w["dim"], w["batch"]
    return {"i8i8": batch * (dim + 4), "f32": batch * dim * 4, "f16": batch * dim * 4,
            "hybrid": batch * dim * 4, "binary": batch * ((dim + 31) // 32) * 4}[w["kind"]]


def measured_traffic(workload, kernel):
    """HBM bytes per launch of `kernel` from the calibrated FETCH_SIZE + WRITE_SIZE counter passes
    summarized in profiles/traffic.json (stored values from rocprofv3 runs, not measured by this
    run; None when this workload has not been profiled)."""
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return None
    entry = json.loads(path.read_text()).get(workload)
    if not entry or entry.get("kernel") != kernel:
        return None
    return entry["traffic_bytes_per_launch"]


def scan_kernel_name(w):
    if w["kind"] == "i8i8" and w["batch"] >= 8:
        return f"mfmaScanKernel<{w['dim'] // 32}, 0>"
    if w["kind"] == "f32" and w["batch"] >= 32 and w["dim"] in (256, 384):
        return f"mfmaSplitScanKernel<{w['dim']}, false>"
    if w["kind"] in ("f32", "f16", "hybrid") and w["batch"] >= 4 and w["dim"] in (128, 256, 384, 512):
        kind = 0 if w["kind"] == "f32" else 1
        lexical = "true" if w["kind"] == "hybrid" else "false"
        return f"mfmaFloatScanKernel<{kind}, {w['dim']}, false, {lexical}>"
    if w["kind"] == "binary" and w["batch"] >= 4 and w["dim"] in (512, 1024):
        # one set of up to 32 queries: the streaming kernel (mode 0: threshold scan); more: the
        # shared-tile kernel
        if w["batch"] <= 32:
            return f"mfmaBinaryStreamKernel<{w['dim'] // 32}, 0>"
        return f"mfmaBinaryScanKernel<{w['dim'] // 32}, false>"
    if w["batch"] <= 4:
        return "singlePassScanKernel"
    return "valuScanKernel"


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


class OracleRunner:
    """The oracle's restatement of the reference's CPU path (tests/cpp/cpu_reference.hpp:12-34: a
    sequential dot per document, then the stable top-k) over the full corpus, for chosen queries
    of a workload: the CPU baseline and the sampled parity checks."""

    def __init__(self, capi, w, corpus, keep, queries):
        import oracle

        self.oracle = oracle
        self.capi, self.w, self.keep = capi, w, keep
        kind = w["kind"]
        log(f"copying the {w['name']} corpus to host for the oracle")
        self.host_q = queries.to_host()[: w["batch"]]
        if kind == "i8i8":
            self.codes = corpus.to_host()
            self.row_scales = keep["scales"].to_host()
        elif kind in ("f16", "hybrid"):
            self.decoded = corpus.to_host().astype(np.float32)
        elif kind == "f32":
            self.decoded = corpus.to_host()
        else:
            self.words = corpus.to_host()
            self.qwords = oracle.pack_binary(self.host_q)

    def rescore_rows(self, ids):
        # the candidates' float16 rows: the 102 GB rescore store does not fit on the host, so the
        # CPU path gathers its C rows per query from the device (about 2% of its time)
        capi, dim, half = self.capi, self.w["dim"], self.keep["rescore"]
        out = np.empty((len(ids), dim), dtype=np.float16)
        for i, r in enumerate(ids):
            capi.call("zcgvs_memcpy_d2h", out[i].ctypes.data, half.ptr + int(r) * dim * 2, dim * 2, None)
        capi.synchronize()
        return out.astype(np.float32)

    def topk(self, rows):
        oracle, w = self.oracle, self.w
        k, n, dim, kind = w["k"], w["n"], w["dim"], w["kind"]
        if kind == "i8i8":
            qcodes, qscales = oracle.quantize_rows_i8(self.host_q[rows])
            return oracle.topk(oracle.scores_i8i8(self.codes, self.row_scales, qcodes, qscales), k)
        if kind == "binary":
            cand, _ = oracle.topk(oracle.scores_hamming(self.words, self.qwords[rows], dim), w["candidates"])
            out_idx = np.empty((len(rows), k), np.int32)
            out_val = np.empty((len(rows), k), np.float32)
            for i, row in enumerate(rows):
                ids = cand[i]
                local, out_val[i] = oracle.topk(
                    oracle.rescore(self.rescore_rows(ids), self.host_q[row:row + 1],
                                   np.arange(len(ids), dtype=np.int32)[None, :]), k)
                out_idx[i] = ids[local[0]]
            return out_idx, out_val
        scores = oracle.scores_f32(self.decoded, self.host_q[rows], oracle.COSINE)
        if kind == "hybrid":
            index, terms = self.keep["index"], self.keep["terms_host"]
            for i, row in enumerate(rows):
                lex = oracle.bm25(index["offsets"], index["posting_docs"], index["posting_weights"], terms[row], n)
                scores[i] = oracle.fuse(scores[i], lex, oracle.max_positive(lex), w["dense_weight"])
        return oracle.topk(scores, k)

    def parity(self, rows, gpu_idx, gpu_val):
        """The sampled queries' GPU top-k against the oracle's: ids and scores bit for bit for the
        integer kinds; ids and the largest relative score difference for the float kinds."""
        ref_idx, ref_val = self.topk(rows)
        got_idx, got_val = gpu_idx[rows], gpu_val[rows]
        if self.w["kind"] == "i8i8":
            return {"queries_checked": len(rows),
                    "bit_exact": bool(np.array_equal(ref_idx, got_idx) and np.array_equal(ref_val, got_val))}
        scale = np.maximum(np.abs(ref_val.astype(np.float64)), 1e-30)
        rel = float(np.max(np.abs(got_val.astype(np.float64) - ref_val) / scale))
        return {"queries_checked": len(rows), "ids_equal": bool(np.array_equal(ref_idx, got_idx)),
                "max_rel_score_diff": float(f"{rel:.3g}")}


def cpu_baseline(runner, gpu_idx, gpu_val, budget_s):
    """The oracle timed on this host for a bounded sample of the workload's queries, with one
    thread and with every core the OpenMP runtime offers (the same per-document sums; results do
    not depend on the thread count). Returns (baseline, parity of the sampled queries)."""
    oracle, w = runner.oracle, runner.w
    batch, n = w["batch"], w["n"]
    all_cores = oracle.threads()
    limit = min(batch, 8) if w["kind"] == "binary" else batch
    variants = []
    rows = []
    for cores, share in ((1, 0.4), (all_cores, 0.6)):
        oracle.set_threads(cores)
        t0 = time.perf_counter()
        runner.topk([0])
        one = time.perf_counter() - t0
        sample = int(max(1, min(limit, share * budget_s / max(one, 1e-6))))
        rows = list(range(sample))
        t0 = time.perf_counter()
        runner.topk(rows)
        elapsed = time.perf_counter() - t0
        variants.append({"cores": cores, "value": round(sample / elapsed, 3), "unit": "queries/s",
                         "queries": sample, "seconds": round(elapsed, 2),
                         "extrapolated": sample < batch})
    oracle.set_threads(all_cores)
    parity = runner.parity(rows, gpu_idx, gpu_val)
    best = variants[-1]
    baseline = {
        "value": best["value"],
        "unit": "queries/s",
        "cores": best["cores"],
        "kind": "port",
        "sample": f"first {best['queries']} of the {batch} queries against all {n:,} rows, "
                  f"{best['seconds']} s on {best['cores']} threads (per-query rate"
                  f"{', extrapolated to the batch' if best['extrapolated'] else ''}); "
                  f"1 thread: {variants[0]['queries']} queries in {variants[0]['seconds']} s",
        "variants": variants,
        "nproc": os.cpu_count(),
        "cpu_model": cpu_model(),
    }
    return baseline, parity


def vendor_yardstick(w, steps: int, warmup: int) -> int:
    """The fp32 score matrix by the vendor BLAS (torch on ROCm calls rocBLAS / hipBLASLt): the
    MI355X analog of the reference's cuBLAS backend (src/cuda/cublas_similarity.cpp:42-49, sgemv at
    batch 1 and sgemm otherwise; fp32, cosine/dot, no mask), timed the way
    apps/bench_kernels.cu:188-208 times it. A yardstick only: it writes the [batch, N] scores and
    selects nothing, so it is not a search step and never the bench's value."""
    import torch

    if w["kind"] != "f32":
        raise SystemExit("bench.py: --vendor-yardstick takes fp32 workloads only (as the reference's cuBLAS backend)")
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(1)
    corpus = torch.randn(w["n"], w["dim"], device=dev, generator=gen)
    corpus /= corpus.norm(dim=1, keepdim=True)
    queries = torch.randn(w["batch"], w["dim"], device=dev, generator=gen)
    queries /= queries.norm(dim=1, keepdim=True)

    def step():
        if w["batch"] == 1:
            return torch.mv(corpus, queries[0])
        return torch.mm(queries, corpus.t())

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for begin, end in events:
        begin.record()
        step()
        end.record()
    torch.cuda.synchronize()
    ms = [begin.elapsed_time(end) for begin, end in events]
    mean = statistics.mean(ms)
    moved = w["n"] * w["dim"] * 4 + w["batch"] * w["n"] * 4  # corpus read + scores written
    print(json.dumps({
        "metric": "vendor fp32 score matrix (torch -> rocBLAS/hipBLASLt), yardstick only",
        "value": round(moved / (mean * 1e-3) / 1e9, 1), "unit": "GB/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "ms_per_step": round(mean, 4), "p50_ms": round(statistics.median(ms), 4),
        "higher_is_better": True, "dtype": "f32", "data": "synthetic (torch.randn rows, L2-normalized)",
        "config": {"workload": w["name"], "N": w["n"], "dim": w["dim"], "batch": w["batch"],
                   "op": "sgemv" if w["batch"] == 1 else "sgemm", "output": "[batch, N] fp32 scores, no top-k"},
    }), flush=True)
    return 0


def measure(capi, w, desc, steps, warmup, graph=False):
    """Times `steps` searches of `desc` (after `warmup`), then, untimed, per-step events (p50) and
    per-phase scan events. Returns the figures and the last result."""
    size = capi.search_workspace_bytes(desc)
    workspace = capi.DeviceArray(size, np.uint8)
    batch, k = desc.batch, desc.k
    out_idx = capi.DeviceArray((batch, k), np.int32)
    out_val = capi.DeviceArray((batch, k), np.float32)
    stream = capi.Stream()
    captured = None
    if graph:
        captured = capi.Graph(stream, lambda: capi.search_topk(desc, workspace, size, out_idx, out_val, stream))

    def step():
        if captured is not None:
            captured.launch(stream)
        else:
            capi.search_topk(desc, workspace, size, out_idx, out_val, stream)

    for _ in range(warmup):
        step()
    stream.synchronize()
    # Timed region: K searches back to back on the stream and nothing else (an event record costs
    # the GPU a few microseconds, comparable to a small search, so none sits between the steps).
    capi.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    stream.synchronize()
    capi.synchronize()
    wall = time.perf_counter() - t0

    # Untimed, after the timed region: the per-step latency (an event pair around every step) and
    # the scan launches' durations (events around each scan launch) from K more searches each.
    max_phases = 8
    starts = [capi.Event() for _ in range(steps)]
    ends = [capi.Event() for _ in range(steps)]
    scan_events = [[capi.Event() for _ in range(2 * max_phases)] for _ in range(steps)]
    for i in range(steps):
        starts[i].record(stream)
        step()
        ends[i].record(stream)
    stream.synchronize()
    phases = 0
    for i in range(steps):
        phases = capi.search_topk_profiled(desc, workspace, size, out_idx, out_val, stream, scan_events[i],
                                           max_phases)
    stream.synchronize()
    used = min(phases, max_phases)
    phase_ms = [[scan_events[i][2 * p].elapsed_ms(scan_events[i][2 * p + 1]) for p in range(used)]
                for i in range(steps)]
    lex_ms = None
    if w["kind"] == "hybrid" and used < max_phases:
        lex_ms = statistics.mean(scan_events[i][2 * used].elapsed_ms(scan_events[i][2 * used + 1])
                                 for i in range(steps))
    flags = np.empty(batch, dtype=np.uint32)
    capi.call("zcgvs_memcpy_d2h", flags.ctypes.data, capi.search_overflow_flags(desc, workspace),
              flags.nbytes, None)
    capi.synchronize()
    result = {
        "wall": wall, "ms_per_step": wall * 1e3 / steps,
        "p50_ms": statistics.median(starts[i].elapsed_ms(ends[i]) for i in range(steps)),
        "phases": phases, "phase_ms": phase_ms, "phase_rows": capi.search_phase_rows(desc, max_phases)[:used],
        "lex_ms": lex_ms, "flags": flags, "idx": out_idx.to_host(), "val": out_val.to_host(),
        "workspace_bytes": size,
    }
    del captured, workspace, out_idx, out_val
    return result


def scan_figures(w, m, keep):
    """The dominant scan kernel's mean launch time and algorithmic bytes, and the step's."""
    steps = len(m["phase_ms"])
    used = len(m["phase_rows"])
    # Dominant kernel: the scan launches of the threshold phases (the MFMA paths compile the dense
    # first phase and the sketch phase as separate kernels; the VALU path runs every phase with one
    # kernel). A sketch plan's last phase is its one full scan.
    first = 1 if scan_kernel_name(w).startswith("mfma") and used > 1 else 0
    launches = list(range(first, used))
    mean_ms = statistics.mean(statistics.mean(m["phase_ms"][i][p] for p in launches) for i in range(steps))
    bytes_launch = statistics.mean(m["phase_rows"][p] * row_bytes(w) + query_bytes(w) for p in launches)
    scan_ms = statistics.mean(sum(m["phase_ms"][i]) for i in range(steps))
    # algorithmic bytes of one step: the corpus once (+ the queries), the lexical stage's postings
    step_bytes = w["n"] * row_bytes(w) + query_bytes(w)
    if w["kind"] == "hybrid":
        step_bytes += lexical_bytes(keep)
    return launches, mean_ms, bytes_launch, scan_ms, step_bytes


def free_all(*arrays):
    for a in arrays:
        if a is not None and hasattr(a, "free"):
            a.free()


def secondary_line(capi, w, key, desc, corpus, keep, queries, steps, warmup, runner=None):
    """One configuration's compact line: step time, roofline fractions, sampled parity."""
    m = measure(capi, w, desc, steps, warmup)
    launches, kernel_ms, bytes_launch, _, step_bytes = scan_figures(w, m, keep)
    line = {
        "workload": key, "name": w["name"], "batch": desc.batch, "k": desc.k,
        "ms_per_step": round(m["ms_per_step"], 4), "p50_ms": round(m["p50_ms"], 4),
        "queries_per_s": round(desc.batch / (m["ms_per_step"] * 1e-3), 1),
        "kernel": scan_kernel_name(w), "launches_per_step": len(launches), "kernel_ms": round(kernel_ms, 4),
        "frac": round(bytes_launch / (kernel_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "step_frac": round(step_bytes / (m["ms_per_step"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "phase_ms": [round(statistics.mean(m["phase_ms"][i][p] for i in range(steps)), 4)
                     for p in range(len(m["phase_rows"]))],
    }
    if m["lex_ms"] is not None:
        lex = lexical_bytes(keep)
        line["lexical_stage"] = {"ms": round(m["lex_ms"], 4), "algorithmic_bytes": lex,
                                 "frac": round(lex / (m["lex_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    if m["flags"].any():
        line["overflow_queries"] = int(m["flags"].sum())
    if runner is None:
        runner = OracleRunner(capi, w, corpus, keep, queries)
    line["parity"] = runner.parity([0] if desc.batch == 1 else [0, desc.batch - 1], m["idx"], m["val"])
    log(f"secondary {key}: {line['ms_per_step']} ms/step, kernel {line['kernel_ms']} ms, frac {line['frac']}, "
        f"parity {line['parity']}")
    return line, runner


def with_batch(capi, desc, batch, k=None):
    """The same search with the first `batch` queries (and k, if given)."""
    d = capi.SearchDesc()
    ctypes = capi.ctypes
    ctypes.memmove(ctypes.byref(d), ctypes.byref(desc), ctypes.sizeof(desc))
    d.batch = batch
    if k is not None:
        d.k = k
    d._owners = list(getattr(desc, "_owners", []))  # the buffers the descriptor points at
    return d


def secondary_runs(capi, steps, warmup, headline_inputs, runner=None):
    """The other benchmark configurations, each a compact line (see secondary_line)."""
    lines = []
    # per-vector int8 10M x 768 at batch 1: the headline's corpus and first query (and the
    # headline's copy of the corpus for the oracle, when it made one)
    w = dict(WORKLOADS["int8-10m-b1"])
    desc, corpus, queries, keep = headline_inputs
    if runner is not None:
        runner.w = w
    line, runner = secondary_line(capi, w, "int8-10m-b1", with_batch(capi, desc, 1), corpus, keep, queries,
                                  steps, warmup, runner)
    lines.append(line)
    del runner
    # float32 5,183 x 384 (the reference's CPU-runnable case)
    w = WORKLOADS["cpu-ref"]
    desc, corpus, queries, keep = build_inputs(capi, w)
    lines.append(secondary_line(capi, w, "cpu-ref", desc, corpus, keep, queries, steps, warmup)[0])
    free_all(corpus, queries)
    # float32 and float16 1M x 384 at batch 1 and 64 (one corpus per type)
    for kind in ("f32", "f16"):
        w64 = WORKLOADS[f"{kind}-1m-b64"]
        desc, corpus, queries, keep = build_inputs(capi, w64)
        line, runner = secondary_line(capi, w64, f"{kind}-1m-b64", desc, corpus, keep, queries, steps, warmup)
        w1 = WORKLOADS[f"{kind}-1m-b1"]
        runner.w = w1
        line1, _ = secondary_line(capi, w1, f"{kind}-1m-b1", with_batch(capi, desc, 1), corpus, keep, queries,
                                  steps, warmup, runner)
        lines += [line1, line]
        del runner
        free_all(corpus, queries)
    # binary 50M x 1024 + float16 rescore of 1000, batch 32
    w = WORKLOADS["binary-50m"]
    desc, corpus, queries, keep = build_inputs(capi, w)
    lines.append(secondary_line(capi, w, "binary-50m", desc, corpus, keep, queries, steps, warmup)[0])
    free_all(corpus, queries, keep.get("rescore"))
    # hybrid BM25 + float16 1M x 384, batch 16
    w = WORKLOADS["hybrid-1m"]
    desc, corpus, queries, keep = build_inputs(capi, w)
    lines.append(secondary_line(capi, w, "hybrid-1m", desc, corpus, keep, queries, steps, warmup)[0])
    free_all(corpus, queries, keep.get("terms"), *keep.get("lexical", {}).values())
    return lines


def reference_tables(capi, steps, warmup):
    """The shapes apps/bench_kernels.cu:151-273 times, on 1M x 384 rows (docs/BENCHMARKS.md)."""
    n, dim = 1_000_000, 384
    out = {}
    stream = capi.Stream()

    def timed(fn):
        for _ in range(warmup):
            fn()
        stream.synchronize()
        events = [(capi.Event(), capi.Event()) for _ in range(steps)]
        for begin, end in events:
            begin.record(stream)
            fn()
            end.record(stream)
        stream.synchronize()
        return statistics.median(begin.elapsed_ms(end) for begin, end in events)

    # storage-type scan: the similarity launcher, one query, cosine, scores [1, N] written
    f32 = capi.DeviceArray((n, dim), np.float32)
    capi.generate_normalized(f32, n, dim, CORPUS_SEED, 0)
    query = capi.DeviceArray((1, dim), np.float32)
    capi.generate_normalized(query, 1, dim, QUERY_SEED, 0)
    capi.synchronize()
    peak = float(np.abs(f32.to_host()).max())
    f16 = capi.DeviceArray((n, dim), np.float16)
    capi.launch_convert_f32_to_f16(f32, f16, n * dim)
    i8 = capi.DeviceArray((n, dim), np.int8)
    scale = peak / 127.0
    capi.launch_convert_f32_to_i8(f32, i8, n * dim, scale)
    words = capi.DeviceArray((n, dim // 32), np.uint32)
    capi.launch_pack_binary(f32, words, n, dim)
    qwords = capi.DeviceArray((1, dim // 32), np.uint32)
    capi.launch_pack_binary(query, qwords, 1, dim)
    scores = capi.DeviceArray((1, n), np.float32)
    capi.synchronize()
    scan = []
    for name, data, dtype, q, row, s in (("float32", f32, capi.F32, query, dim * 4, 1.0),
                                         ("float16", f16, capi.F16, query, dim * 2, 1.0),
                                         ("int8", i8, capi.I8, query, dim, scale),
                                         ("binary", words, capi.BINARY, qwords, dim // 8, 1.0)):
        ms = timed(lambda: capi.launch_similarity(data, dtype, s, n, dim, q, 1, None, capi.COSINE, scores,
                                                  stream))
        moved = n * row
        scan.append({"storage": name, "bytes": moved, "median_ms": round(ms, 4),
                     "gbs": round(moved / (ms * 1e-3) / 1e9, 1),
                     "frac": round(moved / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
    out["similarity_scan_1m_x_384"] = scan
    free_all(f16, i8, words, qwords)

    # top-k over 1M uniform(-1, 1) scores, one query
    rng = np.random.default_rng(11)
    host = rng.uniform(-1.0, 1.0, n).astype(np.float32)
    capi.call("zcgvs_memcpy_h2d", scores.ptr, host.ctypes.data, host.nbytes, None)
    capi.synchronize()
    topk = []
    for k in (10, 100, 1000):
        elems = capi.library().zcgvs_topk_scratch_elements(n, k)
        sa, ia = capi.DeviceArray(elems, np.float32), capi.DeviceArray(elems, np.int32)
        sb, ib = capi.DeviceArray(elems, np.float32), capi.DeviceArray(elems, np.int32)
        oi, ov = capi.DeviceArray(k, np.int32), capi.DeviceArray(k, np.float32)
        ms = timed(lambda: capi.launch_topk(scores, n, k, 1, oi, ov, sa, ia, sb, ib, stream))
        got = oi.to_host()
        expect = np.argsort(-host, kind="stable")[:k]
        topk.append({"k": k, "median_ms": round(ms, 4), "gbs": round(n * 4 / (ms * 1e-3) / 1e9, 1),
                     "ids_equal": bool(np.array_equal(got, expect))})
        free_all(sa, ia, sb, ib, oi, ov)
    out["topk_1m"] = topk
    free_all(scores)

    # the float16 pipeline, k = 100, batch 1, 8, 32, direct and graph replay (fresh corpus copy)
    f16 = capi.DeviceArray((n, dim), np.float16)
    capi.launch_convert_f32_to_f16(f32, f16, n * dim)
    queries = capi.DeviceArray((32, dim), np.float32)
    capi.generate_normalized(queries, 32, dim, 99, 0)
    capi.synchronize()
    free_all(f32, query)
    sweep = []
    w = dict(WORKLOADS["f16-1m-b64"], k=100)
    for batch in (1, 8, 32):
        desc = capi.search_desc(capi.store_desc(f16, n, dim, capi.F16), queries, batch, 100, capi.COSINE)
        row = {"batch": batch}
        for graph in (False, True):
            m = measure(capi, w, desc, steps, warmup, graph=graph)
            tag = "graph" if graph else "direct"
            row[f"{tag}_ms"] = round(m["ms_per_step"], 4)
            row[f"{tag}_queries_per_s"] = round(batch / (m["ms_per_step"] * 1e-3), 1)
        sweep.append(row)
    out["pipeline_f16_1m_k100"] = sweep
    free_all(f16, queries)
    log(f"reference tables: {json.dumps(out)}")
    return out


def main(argv=None) -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--workload", choices=sorted(WORKLOADS), default="int8-10m")
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    parser.add_argument("--no-secondary", action="store_true",
                        help="skip the other configurations and the reference's tables (run by default "
                             "with the default workload only)")
    parser.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU sample work")
    parser.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                        help="before the workload, copy MIB MiB device to device once (a transfer of "
                             "known size for calibrating rocprofv3 FETCH_SIZE/WRITE_SIZE readings)")
    parser.add_argument("--graph", action="store_true",
                        help="time replays of one captured HIP graph of the search instead of direct "
                             "calls (the per-phase kernel times still come from direct calls)")
    parser.add_argument("--no-peak", action="store_true",
                        help="skip the measured HBM read/copy peak (zcgvs_measure_hbm_bandwidth)")
    parser.add_argument("--vendor-yardstick", action="store_true",
                        help="time the fp32 [batch, N] score matrix by the vendor BLAS instead (the analog "
                             "of the reference's cuBLAS backend; fp32 workloads; scores only, no top-k)")
    args = parser.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the corpus would shard by rows, with one gather of batch*k hits per GPU)",
              file=sys.stderr)
        return 2

    if args.vendor_yardstick:
        return vendor_yardstick(WORKLOADS[args.workload], args.steps, args.warmup)

    load_package()
    from zcgvs_amd import capi

    if capi.device_count() <= 0:
        raise SystemExit("bench.py: no HIP device")
    info = capi.device_info(0)
    w = WORKLOADS[args.workload]
    log(f"device {info.name.decode()} {info.arch.decode()} CUs={info.compute_units}; workload {w['name']}")

    if args.copy_probe > 0:
        nbytes = args.copy_probe << 20
        src, dst = capi.DeviceArray(nbytes, np.uint8), capi.DeviceArray(nbytes, np.uint8)
        capi.call("zcgvs_memset", src.ptr, 1, nbytes, None)
        capi.call("zcgvs_memcpy_d2d", dst.ptr, src.ptr, nbytes, None)
        capi.synchronize()
        src.free()
        dst.free()
        log(f"copy probe: {args.copy_probe} MiB device-to-device")
    measured = None
    if not args.no_peak:
        read_gbs, copy_gbs = capi.measure_hbm_bandwidth(4 << 30, 5)
        measured = {"read": round(read_gbs, 1), "copy": round(copy_gbs, 1)}
        log(f"measured HBM: streaming read {read_gbs:.0f} GB/s, copy {copy_gbs:.0f} GB/s "
            f"(nominal {HBM_PEAK_GBS:.0f}, from clocks {info.peak_bandwidth_gbs:.0f})")
    desc, corpus, queries, keep = build_inputs(capi, w)
    log(f"inputs resident; workspace {capi.search_workspace_bytes(desc) / 2**20:.1f} MiB")
    m = measure(capi, w, desc, args.steps, args.warmup, graph=args.graph)
    flags, gpu_idx, gpu_val = m["flags"], m["idx"], m["val"]
    if flags.any():
        # information, not an error: flagged queries took the exact fallback inside the step (the
        # parity check below still compares the sampled results with the oracle)
        log(f"{int(flags.sum())} queries took the exact fallback")

    batch = w["batch"]
    value = batch * args.steps / m["wall"]
    launches, mean_ms, bytes_launch, scan_ms, step_bytes = scan_figures(w, m, keep)
    achieved = bytes_launch / (mean_ms * 1e-3) / 1e9
    phase_rows = m["phase_rows"]
    log("phase ms: " + " ".join(f"{statistics.mean(m['phase_ms'][i][p] for i in range(args.steps)):.3f}"
                                 for p in range(len(phase_rows))) + f"; rows {phase_rows}")
    traffic = measured_traffic(args.workload, scan_kernel_name(w))
    result = {
        "metric": "queries/sec + p50 latency (N=10M d=768 int8, k=100); scan HBM GB/s",
        "value": round(value, 2),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(m["ms_per_step"], 4),
        "p50_ms": round(m["p50_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"i8i8": "int8", "f32": "f32", "f16": "f16", "hybrid": "f16", "binary": "u32"}[w["kind"]],
        "data": "synthetic (seeded N(0,1) rows, L2-normalized, generated on the device)",
        "config": {"workload": w["name"], "N": w["n"], "dim": w["dim"], "batch": batch, "k": w["k"],
                   "scan_phases": m["phases"], "launch": "graph" if args.graph else "direct"},
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": "profiles/traffic.json (calibrated rocprofv3 FETCH_SIZE + WRITE_SIZE of an "
                              "earlier run, not measured by this run)" if traffic is not None else None,
            "kernel": scan_kernel_name(w),
            "launches_per_step": len(launches),
            "kernel_ms": round(mean_ms, 4),
            "algorithmic_bytes_per_launch": int(bytes_launch),
            "all_scan_launches_ms": round(scan_ms, 4),
            "step_algorithmic_bytes": int(step_bytes),
            "step_frac": round(step_bytes / (m["ms_per_step"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        },
    }
    if measured is not None:
        # the same kernel against the rates streaming kernels reach on this device
        result["roofline"]["peak_measured"] = {"read_gbs": measured["read"], "copy_gbs": measured["copy"],
                                               "frac_of_read": round(achieved / measured["read"], 4)}
    result["roofline"]["peak_from_clocks_gbs"] = round(info.peak_bandwidth_gbs, 1)
    if w["kind"] == "hybrid" and m["lex_ms"] is not None:
        lex = lexical_bytes(keep)
        result["lexical_stage"] = {"ms": round(m["lex_ms"], 4), "algorithmic_bytes": lex,
                                   "frac": round(lex / (m["lex_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    if w["kind"] in ("i8i8", "binary") and scan_kernel_name(w).startswith("mfma"):
        # int8 products of codes, or fp4 products of one per bit of a binary row and query
        peak = INT8_MFMA_PEAK_TOPS if w["kind"] == "i8i8" else FP4_MFMA_PEAK_TOPS
        ops = statistics.mean(2.0 * phase_rows[p] * w["dim"] * batch for p in launches)
        tops = ops / (mean_ms * 1e-3) / 1e12
        step_tops = 2.0 * w["n"] * w["dim"] * batch / (m["ms_per_step"] * 1e-3) / 1e12
        result["mfma"] = {"achieved": round(tops, 1), "peak": peak, "unit": "TOP/s",
                          "frac": round(tops / peak, 4), "step_frac": round(step_tops / peak, 4)}
    if flags.any():
        result["overflow_queries"] = int(flags.sum())
    runner = None
    if not args.no_cpu:
        runner = OracleRunner(capi, w, corpus, keep, queries)
        baseline, parity = cpu_baseline(runner, gpu_idx, gpu_val, args.cpu_budget)
        result["cpu_baseline"] = baseline
        result["parity"] = parity
    if not args.no_secondary and args.workload == "int8-10m":
        t0 = time.perf_counter()
        result["secondary"] = secondary_runs(capi, args.steps, args.warmup, (desc, corpus, queries, keep), runner)
        runner = None
        free_all(corpus, queries, keep.get("scales"))
        result["reference_tables"] = reference_tables(capi, args.steps, args.warmup)
        log(f"secondary lines and reference tables: {time.perf_counter() - t0:.1f} s")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
