"""CPU checks of bench.py's contract that need no GPU: the multi-GPU refusal
and the figures it reads from the committed rocprofv3 summary."""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_profile_figures_match_the_committed_summary():
    text = open(bench.TRAFFIC_FILE).read()
    fig = bench.read_profile_figures()
    # the summary states the scaled read and write bytes it adds up
    assert fig["traffic"] == 335824365 + 67108864
    assert f"hbm_bytes_per_launch: {int(fig['traffic'])}" in text
    assert fig["mfma_busy_pct"] == 61.9 and fig["lds_bank_conflict_pct"] == 0.29
    # the counters name the workload they were measured on
    assert fig["counters_workload"].startswith("ns_h8 (B1 H8 Sq=Skv=16384 D128")


def test_conv_profile_traffic_is_read():
    fig = bench.read_profile_figures(bench.CONV_TRAFFIC_FILE)
    assert fig["traffic"] == 217144832 + 23617536
