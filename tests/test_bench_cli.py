"""bench.py's argument checks, which end before any device work: more than one GPU is refused with
the sharding note, and the vendor BLAS yardstick takes fp32 workloads only (the reference's cuBLAS
backend covers fp32 alone, src/cuda/cublas_similarity.cpp:15-20)."""

import sys
from pathlib import Path

import pytest

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused(capsys):
    assert bench.main(["--gpus", "2"]) == 2
    assert "one GPU" in capsys.readouterr().err


@pytest.mark.parametrize("workload", ["int8-10m", "f16-1m-b1", "binary-50m"])
def test_vendor_yardstick_takes_fp32_only(workload):
    with pytest.raises(SystemExit, match="fp32 workloads only"):
        bench.main(["--workload", workload, "--vendor-yardstick"])
