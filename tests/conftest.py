import importlib.util
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "zero-copy-gpu-vector-search-re-ranking-engine_amd"


def _load_package():
    if "zcgvs_amd" in sys.modules:
        return sys.modules["zcgvs_amd"]
    spec = importlib.util.spec_from_file_location("zcgvs_amd", PKG / "__init__.py",
                                                  submodule_search_locations=[str(PKG)])
    module = importlib.util.module_from_spec(spec)
    sys.modules["zcgvs_amd"] = module
    spec.loader.exec_module(module)
    return module


_load_package()
for path in (str(ROOT), str(PKG)):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) to run")


@pytest.fixture(scope="session")
def capi():
    from zcgvs_amd import capi as module
    module.library()
    return module


@pytest.fixture(scope="session")
def gpu(capi):
    # A test marked gpu needs a HIP device; without one it fails rather than passing vacuously.
    if capi.device_count() <= 0:
        pytest.fail("no HIP device visible to a test marked gpu")
    return capi
