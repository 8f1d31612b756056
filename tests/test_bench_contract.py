"""The parts of bench.py's contract that need no GPU.

* More than one GPU is refused with a message (this build measures one GPU).
* Without a ROCm device the bench refuses to run rather than timing a CPU path.
* Every workload's roofline finds its HBM traffic figure (the rocprofv3
  FETCH_SIZE / WRITE_SIZE summary) in the committed profiles, at or above the
  algorithmic bytes its kernel must move.
"""

from __future__ import annotations

import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*args):
    return subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), *args], capture_output=True, text=True,
                          timeout=300, check=False)


def test_more_than_one_gpu_is_refused():
    r = _bench("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_refuses_without_a_gpu():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present: the bench would run")
    r = _bench("--workload", "copy", "--steps", "1", "--warmup", "0")
    assert r.returncode == 2
    assert "needs a ROCm GPU" in r.stderr


# (kernel, profile constant, algorithmic bytes per launch or None where the
# figure is not byte-bound)
TRAFFIC = [
    ("materialize_tiles_tr8", "TRAFFIC_PROFILE", None),  # MFMA-bound: the bytes the L2 side moves
    ("score_ring64", "TRAFFIC_PROFILE", (128 + 64) * 218_112_000 * 2.0),  # 16 train blocks of 8 per pass
    ("ghost_gram_tiles_v3", "GHOST_TRAFFIC", None),
    ("da_project_outer", "PROJECT_TRAFFIC", 640 * 128 * (4096 + 11008) * 2.0),
    ("ghost_grouped_tiles_v3", "MOE_TRAFFIC", None),
    ("da_project_outer", "CAPTURE_TRAFFIC", None),
    ("score_ring64", "STORE_TRAFFIC", (4096 + 128) * 3 * 4096 * 2.0),
    ("materialize_tiles_tr", "KFAC_TRAFFIC", None),
]


@pytest.mark.parametrize(("kernel", "profile", "algorithmic"), TRAFFIC)
def test_profiles_hold_each_rooflines_traffic(kernel, profile, algorithmic):
    import bench

    path = getattr(bench, profile)
    got = bench.profiled_traffic(kernel, path)
    assert got is not None, f"{os.path.relpath(path, REPO)} has no traffic_per_launch line for {kernel}"
    assert got > 0
    if algorithmic is not None:
        # HBM bytes can only exceed what the kernel must read and write once
        assert got >= 0.99 * algorithmic, (kernel, got, algorithmic)


def test_missing_profile_reads_as_none(tmp_path):
    import bench

    assert bench.profiled_traffic("materialize_tiles_tr8", str(tmp_path / "absent.md")) is None
