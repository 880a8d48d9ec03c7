"""bench.py on the CPU: the one-GPU guard and the algorithmic byte model
behind `roofline.achieved`.

* `--gpus N` with N > 1 exits with status 2 and says why, before touching
  torch or a GPU;
* the active-pixel counts equal an independent numpy count of the reference's
  mask (r^2 + c^2 <= radius^2; the scatters also skip column 0 of the rows
  i >= n/2);
* the headline's bytes per launch are the documented figures:
  2048 * 25844 * 72 + 2048 * 7180 * 8 for the forward and
  2048 * 25716 * 108 + 12 * 512 * 512 * 257 for the backprojection.
"""
import os
import subprocess
import sys

import numpy as np
import pytest

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def _numpy_counts(n, cutoff):
    radius = n / 2.0 if cutoff is None else float(cutoff)
    i = np.arange(n)[:, None]
    r = np.where(i <= n // 2, i, i - n)
    c = np.arange(n // 2 + 1)[None, :]
    active = r * r + c * c <= radius * radius
    scatter = active & ~((c == 0) & (i >= n // 2))
    return active.size, int(active.sum()), int(scatter.sum())


@pytest.mark.parametrize("n,cutoff", [(8, None), (9, None), (64, None), (64, 10.5), (128, 64.0), (256, None),
                                      (256, 64.0), (255, 200.0)])
def test_active_counts_match_numpy(n, cutoff):
    assert bench.active_counts(n, cutoff) == _numpy_counts(n, cutoff)


def test_headline_bytes_per_launch():
    total, fwd, bwd = bench.active_counts(256)
    assert (total, fwd, bwd) == (256 * 129, 25844, 25716)
    assert bench.bytes_forward(2048, 256, 3, "linear") == 2048 * 25844 * 72 + 2048 * 7180 * 8
    assert bench.bytes_backproject(2048, 256, 3, "linear", 512 * 512 * 257, True) == \
        2048 * 25716 * 108 + 12 * 512 * 512 * 257
    assert abs(bench.bytes_forward(2048, 256, 3, "linear") / 1e9 - 3.928) < 5e-4
    assert abs(bench.bytes_backproject(2048, 256, 3, "linear", 512 * 512 * 257, True) / 1e9 - 6.496) < 5e-4


def test_compulsory_bytes_of_the_headline():
    """Each input read once and each output written once: the forward reads the 512 x 512 x 257
    complex64 volume (0.539 GB) and writes 2048 projections of 256 x 129 (0.541 GB); the weighted
    backprojection reads projections and weights and writes the data and weight volumes."""
    V, S = 512 * 512 * 257, 2048 * 256 * 129
    assert bench.compulsory_forward(S, V) == 8 * V + 8 * S
    assert abs(bench.compulsory_forward(S, V) / 1e9 - (0.539 + 0.541)) < 2e-3
    assert bench.compulsory_backproject(S, V, True) == 12 * S + 12 * V
    assert bench.compulsory_backproject(S, V, False) == 8 * S + 8 * V


def test_euler_rotations_are_rotations():
    import torch
    R = bench.euler_rotations(2, 7, torch.Generator().manual_seed(3)).double()
    eye = torch.eye(3, dtype=torch.float64)
    assert (R @ R.transpose(-1, -2) - eye).abs().max() < 1e-6
    assert (torch.linalg.det(R) - 1).abs().max() < 1e-6


def test_measured_traffic_reads_the_commit_stamp(tmp_path, monkeypatch):
    prof = tmp_path / "profiles"
    prof.mkdir()
    (prof / "hbm_traffic_x.md").write_text('measured_at_commit: abc1234\n'
                                           'traffic_bytes_per_call: {"op": 1000.0}\n')
    monkeypatch.setattr(bench.os.path, "abspath", lambda p: str(tmp_path / "bench.py"))
    per_op, commit = bench.measured_traffic("x")
    assert per_op == {"op": 1000.0} and commit == "abc1234"
