"""MI355X-native (gfx950) zero-copy search hot path.

Layout:
    csrc/         HIP kernels and the C ABI (include/zcgvs_hip.h) -> lib/libzcgvs_hip.so
    host/         C++17 host: Searcher, EmbeddingStore, LexicalIndex, Engine -> lib/libzcgvs.so
    bindings/     pybind11 module `zcgvs_engine` (the reference's Python names)
    zcgvs_tools/  on-disk formats (ZCVE/ZCVM/ZCVL) and synthetic data helpers
    capi.py       ctypes binding of the C ABI
    build.py      in-tree build

The directory name is not a Python identifier; load it with `load_package()` from
__graft_entry__.py (importlib under the name `zcgvs_amd`), or put this directory on sys.path to
import `zcgvs_engine` and `zcgvs_tools` directly.
"""

from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
LIB_DIR = PACKAGE_DIR / "lib"
HIP_LIBRARY = LIB_DIR / "libzcgvs_hip.so"
HOST_LIBRARY = LIB_DIR / "libzcgvs.so"
