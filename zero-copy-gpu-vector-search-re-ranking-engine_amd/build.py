"""Builds the native parts of the package in-tree.

    lib/libzcgvs_hip.so      HIP kernels + the C ABI of include/zcgvs_hip.h (hipcc, gfx950)
    lib/libzcgvs.so          C++17 host: Searcher, EmbeddingStore, LexicalIndex, Engine
                             (g++; reaches the GPU only through libzcgvs_hip.so)
    zcgvs_engine*.so         pybind11 module with the reference's Python names

Usage: python build.py [--jobs N] [--only hip|host|bindings] [--roctx]

--roctx (or ZCGVS_WITH_ROCTX=1) compiles the host's profiler ranges in (include/zcgvs/core/
trace_range.hpp) and links librocprofiler-sdk-roctx; the default build has no profiler dependency.
"""

from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
INCLUDE = ROOT / "include"
LIB = PKG / "lib"
OBJ = PKG / "_build"
ARCH = os.environ.get("ZCGVS_OFFLOAD_ARCH", "gfx950")

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")

# Packed FP32 instructions are disabled for every HIP translation unit (the host pass warns
# that it does not know the feature; that warning is harmless).
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{PKG / 'csrc'}",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", f"-I{INCLUDE}"]


def _run(cmd: list[str]) -> None:
    result = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    stderr = "\n".join(line for line in result.stderr.splitlines() if noise not in line)
    if result.returncode != 0:
        raise RuntimeError(f"command failed ({result.returncode}): {' '.join(cmd)}\n{stderr}")
    if stderr.strip():
        print(stderr, file=sys.stderr)


def _compile_all(jobs: list[list[str]], workers: int) -> None:
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        for future in [pool.submit(_run, job) for job in jobs]:
            future.result()


def build_hip(workers: int) -> Path:
    OBJ.mkdir(exist_ok=True)
    LIB.mkdir(exist_ok=True)
    sources = sorted((PKG / "csrc").glob("*.hip"))
    objects = [OBJ / (src.stem + ".hip.o") for src in sources]
    _compile_all([[HIPCC, *HIP_FLAGS, "-c", str(s), "-o", str(o)] for s, o in zip(sources, objects)],
                 workers)
    target = LIB / "libzcgvs_hip.so"
    tmp = target.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)])
    os.replace(tmp, target)
    return target


def build_host(workers: int, roctx: bool = False) -> Path | None:
    sources = sorted((PKG / "host").glob("*.cpp"))
    if not sources:
        return None
    OBJ.mkdir(exist_ok=True)
    objects = [OBJ / (src.stem + ".host.o") for src in sources]
    trace = ["-DZCGVS_WITH_ROCTX", f"-I{ROCM}/include"] if roctx else []
    _compile_all([[CXX, *CXX_FLAGS, *trace, "-c", str(s), "-o", str(o)] for s, o in zip(sources, objects)],
                 workers)
    target = LIB / "libzcgvs.so"
    tmp = target.with_suffix(".so.tmp")
    trace_lib = [f"-L{ROCM}/lib", "-lrocprofiler-sdk-roctx", f"-Wl,-rpath,{ROCM}/lib"] if roctx else []
    _run([CXX, "-shared", "-fPIC", *map(str, objects), "-o", str(tmp), f"-L{LIB}", "-lzcgvs_hip",
          *trace_lib, "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, target)
    return target


def build_bindings() -> Path | None:
    source = PKG / "bindings" / "module.cpp"
    if not source.exists():
        return None
    import pybind11

    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    target = PKG / f"zcgvs_engine{suffix}"
    tmp = target.with_suffix(".tmp")
    _run([CXX, *CXX_FLAGS, "-shared", "-fvisibility=hidden", f"-I{pybind11.get_include()}",
          f"-I{sysconfig.get_paths()['include']}", str(source), "-o", str(tmp), f"-L{LIB}",
          "-lzcgvs", "-lzcgvs_hip", "-Wl,-rpath,$ORIGIN/lib"])
    os.replace(tmp, target)
    return target


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 4))
    parser.add_argument("--only", choices=["hip", "host", "bindings"], default=None)
    parser.add_argument("--roctx", action="store_true", default=os.environ.get("ZCGVS_WITH_ROCTX") == "1",
                        help="compile the host's roctx profiler ranges in")
    args = parser.parse_args(argv)
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise SystemExit(f"hipcc not found at {HIPCC}")
    if args.only in (None, "hip"):
        print("built", build_hip(args.jobs))
    if args.only in (None, "host"):
        built = build_host(args.jobs, args.roctx)
        if built:
            print("built", built)
    if args.only in (None, "bindings"):
        built = build_bindings()
        if built:
            print("built", built)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
