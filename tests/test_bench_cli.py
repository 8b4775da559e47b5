"""CPU checks of bench.py's contract that need no GPU: the multi-GPU refusal
and the figures it reads from the committed rocprofv3 summary."""

import os
import re
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


def _scaled_bytes(text, what):
    """The '<what> = N KiB * 1024 * f = B B' line of the summary, checked."""
    m = re.search(rf"^\s*{what}\s*=\s*([\d,.]+) KiB \* 1024 \* ([\d.]+)\s*=\s*([\d,]+) B",
                  text, re.M)
    assert m, what
    kib, factor, total = (float(m.group(1).replace(",", "")), float(m.group(2)),
                          int(m.group(3).replace(",", "")))
    assert abs(kib * 1024 * factor - total) <= 0.5e-4 * total
    return total


def test_profile_figures_match_the_committed_summary():
    text = open(bench.TRAFFIC_FILE).read()
    fig = bench.read_profile_figures()
    # the summary states the scaled read and write bytes it adds up
    read, write = _scaled_bytes(text, "read"), _scaled_bytes(text, "write")
    assert fig["traffic"] == read + write
    assert f"hbm_bytes_per_launch: {int(fig['traffic'])}" in text
    # O (16 heads x 16384 rows x 128 dims fp16) is written exactly once
    assert write == 16 * 16384 * 128 * 2
    # reads: at least Q, K and V once
    assert read >= 3 * 16 * 16384 * 128 * 2
    assert 40 < fig["mfma_busy_pct"] < 100 and 0 <= fig["lds_bank_conflict_pct"] < 5
    # the counters name the workload they were measured on
    assert fig["counters_workload"].startswith("ns_h8 (B1 H8 Sq=Skv=16384 D128")


def test_driver_form_reconciliation_is_consistent():
    """The driver-form figures bench.py reports: useful = busy x 32/34, and
    useful x SQ clock / 2.4 GHz reproduces the measured frac within 1 %."""
    fig = bench.read_driver_form_figures()
    assert fig is not None and all(fig[k] is not None for k in
                                   ("sq_clock_ghz", "mfma_busy_pct", "useful_mfma_pct",
                                    "predicted_frac", "measured_frac"))
    assert abs(fig["mfma_busy_pct"] * 32 / 34 - fig["useful_mfma_pct"]) < 0.1
    pred = fig["useful_mfma_pct"] / 100 * fig["sq_clock_ghz"] / 2.4
    assert abs(pred - fig["predicted_frac"]) < 2e-3
    assert abs(fig["predicted_frac"] / fig["measured_frac"] - 1) < 0.01


def test_conv_profile_traffic_is_read():
    fig = bench.read_profile_figures(bench.CONV_TRAFFIC_FILE)
    assert fig["traffic"] == 217144832 + 23617536


def test_warm_up_count(monkeypatch):
    """An explicit --warmup is run exactly; the default sizes the count to
    about WARMUP_MS of launches from one timed launch, within its bounds."""
    import time

    import torch

    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
    calls = []

    def launch(ms):
        def call():
            calls.append(1)
            time.sleep(ms * 1e-3)
        return call

    assert bench.warm_up(launch(0), 7) == 7 and len(calls) == 7
    calls.clear()
    n = bench.warm_up(launch(5), None)  # ~50 launches of 5 ms
    assert n == len(calls)
    assert bench.MIN_WARMUP <= n <= bench.WARMUP_MS / 5 + 1
    calls.clear()
    assert bench.warm_up(launch(20), None) == bench.MIN_WARMUP == len(calls)
