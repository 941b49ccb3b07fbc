"""bench.py's command line, without a GPU: runs on more than one GPU are refused with a message
(the engine runs on one GPU), and the FLOP counts the MFMA-bound workloads report reproduce the
published per-phase totals (3756.15 GFLOP per prefill, 660.53 GFLOP per vision call)."""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_flop_counts_match_the_published_phase_totals():
    assert round(bench.prefill_flops(18, 1, 968) / 1e9, 2) == 3756.15
    assert round(bench.vision_flops(27, 3) / 1e9, 2) == 660.53
