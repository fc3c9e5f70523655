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
Other workloads: --workload {int8-10m, f32-1m-b1, f16-1m-b1, f32-1m-b64, f16-1m-b64,
binary-50m, cpu-ref}.

Prints one JSON line: queries/s over the timed steps, p50 step latency, the scan kernel's
roofline (algorithmic bytes / scan time, from events around the scan launches), and the CPU
oracle timed on a bounded sample of the same queries on this host (with a full-size parity
check of the sampled queries against the GPU result).
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
        keep["postings"] = int(index["offsets"][-1])
        keep["index"] = index
        keep["terms_host"] = terms
        extra.update(lex_offsets=keep["lexical"]["offsets"], lex_docs=keep["lexical"]["posting_docs"],
                     lex_weights=keep["lexical"]["posting_weights"], lex_doc_count=n,
                     lex_vocab_size=w["vocab"], query_terms=keep["terms"], lexical_stride=w["terms"],
                     dense_weight=w["dense_weight"], flags=capi.SEARCH_SORTED_POSTINGS)
    desc = capi.search_desc(store, queries, batch, w["k"], capi.COSINE, **extra)
    return desc, corpus, queries, keep


def row_bytes(w):
    """Algorithmic HBM bytes per corpus row a scan reads (row + its per-row scale)."""
    dim = w["dim"]
    if w["kind"] == "hybrid":
        return dim * 2 + 4 * w["batch"]  # the row and its fused lexical score per query
    return {"i8i8": dim + 4, "f32": dim * 4, "f16": dim * 2, "binary": (dim + 31) // 32 * 4}[w["kind"]]


def query_bytes(w):
    """Bytes of the (device-prepared) queries one scan launch reads."""
    dim, batch = w["dim"], w["batch"]
    return {"i8i8": batch * (dim + 4), "f32": batch * dim * 4, "f16": batch * dim * 4,
            "hybrid": batch * dim * 4, "binary": batch * ((dim + 31) // 32) * 4}[w["kind"]]


def measured_traffic(workload, kernel):
    """HBM bytes per launch of `kernel` from the calibrated FETCH_SIZE + WRITE_SIZE counter passes
    summarized in profiles/ (None when this workload has not been profiled)."""
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
        # up to 32 queries per launch: the streaming kernel; more: the shared-tile kernel
        name = "mfmaBinaryStreamKernel" if w["batch"] <= 32 else "mfmaBinaryScanKernel"
        return f"{name}<{w['dim'] // 32}, false>"
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


def cpu_baseline(capi, w, corpus, keep, queries, gpu_idx, gpu_val, budget_s):
    """The oracle's restatement of the reference's CPU path (tests/cpp/cpu_reference.hpp:12-34:
    a sequential dot per document, then the stable top-k) over the full corpus for a bounded
    sample of the same queries, timed on this host with one thread and with every core the
    OpenMP runtime offers (the same per-document sums; results do not depend on the thread
    count). Returns (baseline, parity of the sampled queries against the GPU result)."""
    import oracle

    n, dim, batch, k = w["n"], w["dim"], w["batch"], w["k"]
    kind = w["kind"]
    log("copying corpus to host for the CPU baseline")
    host_q = queries.to_host()
    if kind == "i8i8":
        codes = corpus.to_host()
        row_scales = keep["scales"].to_host()
    elif kind in ("f16", "hybrid"):
        decoded = corpus.to_host().astype(np.float32)
    elif kind == "f32":
        decoded = corpus.to_host()
    else:
        words = corpus.to_host()
        qwords = oracle.pack_binary(host_q)
        half = keep["rescore"]

    def rescore_rows(ids):
        # the candidates' float16 rows: the 102 GB rescore store does not fit on the host, so the
        # CPU path gathers its C rows per query from the device (about 2% of its time)
        out = np.empty((len(ids), dim), dtype=np.float16)
        for i, r in enumerate(ids):
            capi.call("zcgvs_memcpy_d2h", out[i].ctypes.data, half.ptr + int(r) * dim * 2, dim * 2, None)
        capi.synchronize()
        return out.astype(np.float32)

    def run(rows):
        if kind == "i8i8":
            qcodes, qscales = oracle.quantize_rows_i8(host_q[rows])
            return oracle.topk(oracle.scores_i8i8(codes, row_scales, qcodes, qscales), k)
        if kind == "binary":
            cand, _ = oracle.topk(oracle.scores_hamming(words, qwords[rows], dim), w["candidates"])
            out_idx = np.empty((len(rows), k), np.int32)
            out_val = np.empty((len(rows), k), np.float32)
            for i, row in enumerate(rows):
                ids = cand[i]
                local, out_val[i] = oracle.topk(
                    oracle.rescore(rescore_rows(ids), host_q[row:row + 1], np.arange(len(ids), dtype=np.int32)[None, :]), k)
                out_idx[i] = ids[local[0]]
            return out_idx, out_val
        scores = oracle.scores_f32(decoded, host_q[rows], oracle.COSINE)
        if kind == "hybrid":
            index, terms = keep["index"], keep["terms_host"]
            for i, row in enumerate(rows):
                lex = oracle.bm25(index["offsets"], index["posting_docs"], index["posting_weights"], terms[row], n)
                scores[i] = oracle.fuse(scores[i], lex, oracle.max_positive(lex), w["dense_weight"])
        return oracle.topk(scores, k)

    all_cores = oracle.threads()
    limit = min(batch, 8) if kind == "binary" else batch
    variants = []
    results = None
    for cores, share in ((1, 0.4), (all_cores, 0.6)):
        oracle.set_threads(cores)
        t0 = time.perf_counter()
        run([0])
        one = time.perf_counter() - t0
        sample = int(max(1, min(limit, share * budget_s / max(one, 1e-6))))
        rows = list(range(sample))
        t0 = time.perf_counter()
        got = run(rows)
        elapsed = time.perf_counter() - t0
        variants.append({"cores": cores, "value": round(sample / elapsed, 3), "unit": "queries/s",
                         "queries": sample, "seconds": round(elapsed, 2),
                         "extrapolated": sample < batch})
        results = (rows, got)
    oracle.set_threads(all_cores)
    rows, (ref_idx, ref_val) = results
    sample = len(rows)
    exact_kind = kind == "i8i8"
    if exact_kind:
        equal = bool(np.array_equal(ref_idx, gpu_idx[:sample]) and np.array_equal(ref_val, gpu_val[:sample]))
    else:
        equal = bool(np.array_equal(ref_idx, gpu_idx[:sample]))
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
    parity = {"queries_checked": sample, "bit_exact" if exact_kind else "ids_equal": equal}
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


def main(argv=None) -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--workload", choices=sorted(WORKLOADS), default="int8-10m")
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
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
    size = capi.search_workspace_bytes(desc)
    workspace = capi.DeviceArray(size, np.uint8)
    out_idx = capi.DeviceArray((w["batch"], w["k"]), np.int32)
    out_val = capi.DeviceArray((w["batch"], w["k"]), np.float32)
    stream = capi.Stream()
    log(f"inputs resident; workspace {size / 2**20:.1f} MiB")

    graph = None
    if args.graph:
        graph = capi.Graph(stream, lambda: capi.search_topk(desc, workspace, size, out_idx, out_val, stream))

    def step():
        if graph is not None:
            graph.launch(stream)
        else:
            capi.search_topk(desc, workspace, size, out_idx, out_val, stream)

    for _ in range(args.warmup):
        step()
    stream.synchronize()

    # Timed region: K searches back to back on the stream and nothing else (an event record costs
    # the GPU a few microseconds, comparable to a small search, so none sits between the steps).
    capi.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    stream.synchronize()
    capi.synchronize()
    wall = time.perf_counter() - t0

    # Untimed, after the timed region: the per-step latency (an event pair around every step) and
    # the scan launches' durations (events around each scan launch) from K more searches each.
    max_phases = 8
    starts = [capi.Event() for _ in range(args.steps)]
    ends = [capi.Event() for _ in range(args.steps)]
    scan_events = [[capi.Event() for _ in range(2 * max_phases)] for _ in range(args.steps)]
    for i in range(args.steps):
        starts[i].record(stream)
        step()
        ends[i].record(stream)
    stream.synchronize()
    for i in range(args.steps):
        phases = capi.search_topk_profiled(desc, workspace, size, out_idx, out_val, stream,
                                           scan_events[i], max_phases)
    stream.synchronize()

    step_ms = [starts[i].elapsed_ms(ends[i]) for i in range(args.steps)]
    used = min(phases, max_phases)
    phase_ms = [[scan_events[i][2 * p].elapsed_ms(scan_events[i][2 * p + 1]) for p in range(used)]
                for i in range(args.steps)]
    phase_rows = capi.search_phase_rows(desc, max_phases)[:used]
    flags = np.empty(w["batch"], dtype=np.uint32)
    capi.call("zcgvs_memcpy_d2h", flags.ctypes.data, capi.search_overflow_flags(desc, workspace),
              flags.nbytes, None)
    capi.synchronize()
    if flags.any():
        # information, not an error: flagged queries took the exact fallback inside the step (the
        # parity check below still compares the sampled results with the oracle)
        log(f"{int(flags.sum())} queries took the exact fallback")
    gpu_idx, gpu_val = out_idx.to_host(), out_val.to_host()

    batch = w["batch"]
    value = batch * args.steps / wall
    # Dominant kernel: the scan launches of the threshold phases (the MFMA paths compile the dense
    # first phase as a separate kernel; the VALU path runs every phase with one kernel).
    first = 1 if scan_kernel_name(w).startswith("mfma") and used > 1 else 0
    launches = list(range(first, used))
    mean_ms = statistics.mean(statistics.mean(phase_ms[i][p] for p in launches) for i in range(args.steps))
    bytes_launch = statistics.mean(phase_rows[p] * row_bytes(w) + query_bytes(w) for p in launches)
    achieved = bytes_launch / (mean_ms * 1e-3) / 1e9
    scan_ms = statistics.mean(sum(phase_ms[i]) for i in range(args.steps))
    log("phase ms: " + " ".join(f"{statistics.mean(phase_ms[i][p] for i in range(args.steps)):.3f}"
                                 for p in range(used)) + f"; rows {phase_rows}")
    result = {
        "metric": "queries/sec + p50 latency (N=10M d=768 int8, k=100); scan HBM GB/s",
        "value": round(value, 2),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "p50_ms": round(statistics.median(step_ms), 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"i8i8": "int8", "f32": "f32", "f16": "f16", "hybrid": "f16", "binary": "u32"}[w["kind"]],
        "data": "synthetic (seeded N(0,1) rows, L2-normalized, generated on the device)",
        "config": {"workload": w["name"], "N": w["n"], "dim": w["dim"], "batch": batch, "k": w["k"],
                   "scan_phases": phases, "launch": "graph" if graph is not None else "direct"},
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(args.workload, scan_kernel_name(w)),
            "kernel": scan_kernel_name(w),
            "launches_per_step": len(launches),
            "kernel_ms": round(mean_ms, 4),
            "algorithmic_bytes_per_launch": int(bytes_launch),
            "all_scan_launches_ms": round(scan_ms, 4),
        },
    }
    if measured is not None:
        # the same kernel against the rates streaming kernels reach on this device
        result["roofline"]["peak_measured"] = {"read_gbs": measured["read"], "copy_gbs": measured["copy"],
                                               "frac_of_read": round(achieved / measured["read"], 4)}
    result["roofline"]["peak_from_clocks_gbs"] = round(info.peak_bandwidth_gbs, 1)
    if w["kind"] == "i8i8" and scan_kernel_name(w).startswith("mfma"):
        ops = statistics.mean(2.0 * phase_rows[p] * w["dim"] * batch for p in launches)
        tops = ops / (mean_ms * 1e-3) / 1e12
        result["mfma"] = {"achieved": round(tops, 1), "peak": INT8_MFMA_PEAK_TOPS, "unit": "TOP/s",
                          "frac": round(tops / INT8_MFMA_PEAK_TOPS, 4)}
    if flags.any():
        result["overflow_queries"] = int(flags.sum())
    if not args.no_cpu:
        baseline, parity = cpu_baseline(capi, w, corpus, keep, queries, gpu_idx, gpu_val, args.cpu_budget)
        result["cpu_baseline"] = baseline
        if parity is not None:
            result["parity"] = parity
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
