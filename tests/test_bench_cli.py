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


def test_lexical_stage_is_priced_by_postings():
    # 8 B per posting of every query's terms (repeated terms counted per query) + 16 B of offsets
    # per term; the [batch, N] lexical score matrix is not work
    import numpy as np
    offsets = np.array([0, 5, 5, 12, 20], dtype=np.int64)
    keep = {"index": {"offsets": offsets}, "terms_host": np.array([[0, 2, -1], [2, 3, 1]], dtype=np.int32)}
    assert bench.lexical_bytes(keep) == (5 + 7 + 7 + 8 + 0) * 8 + 5 * 16
    w = dict(bench.WORKLOADS["hybrid-1m"])
    assert bench.row_bytes(w) == 2 * w["dim"]


def test_with_batch_keeps_the_descriptor(capi):
    corpus = capi.store_desc(1 << 20, 1000, 64, capi.F32)
    desc = capi.search_desc(corpus, 1 << 21, 64, 10, capi.DOT, flags=capi.SEARCH_SORTED_POSTINGS)
    one = bench.with_batch(capi, desc, 1, k=100)
    assert (one.batch, one.k, desc.batch, desc.k) == (1, 100, 64, 10)
    assert one.corpus.data == desc.corpus.data and one.queries == desc.queries
    assert one.metric == capi.DOT and one.flags == capi.SEARCH_SORTED_POSTINGS
