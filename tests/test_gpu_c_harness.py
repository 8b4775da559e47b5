"""The C ABI without torch: gfx906_amd/lib/launch_harness (built by
gfx906_amd/build.py from gfx906_amd/csrc/launch_harness.cpp) hipMallocs its
own buffers, calls launch() on stream 0 and times it with hipEvents, as the
reference's micro3.hip does (micro3.hip:4-17). The test hands it fp16 inputs
as raw files and checks its output file at the north-star bar: the committed
golden fixtures against their float64 outputs, and one VAE-sized head (which
launch() splits over the static scratch) against SDPA MATH on seeded rows."""

import json
import os
import subprocess

import numpy as np
import pytest
import torch

from gfx906_amd.build import HARNESS
from oracle.attention import MAX_ABS_TOL, MEAN_ABS_TOL, error_stats, make_inputs, sdpa_math_fp32

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "attn_golden.npz")


def run_harness(tmp_path, q, k, v, scale, reps):
    """q, k, v: fp16 numpy arrays [B,H,S,D]; returns (o fp16 array, timing dict)."""
    assert HARNESS.is_file(), f"{HARNESS} not built; run python -m gfx906_amd.build"
    B, H, Sq, D = q.shape
    Skv = k.shape[2]
    for name, x in (("q", q), ("k", k), ("v", v)):
        np.ascontiguousarray(x, dtype=np.float16).tofile(tmp_path / f"{name}.bin")
    res = subprocess.run([str(HARNESS), str(tmp_path), str(B), str(H), str(Sq), str(Skv), str(D),
                          repr(float(scale)), str(reps)],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    o = np.fromfile(tmp_path / "o.bin", dtype=np.float16).reshape(B, H, Sq, D)
    return o, json.loads(res.stdout.strip().splitlines()[-1])


def golden_cases():
    z = np.load(GOLDEN)
    return sorted({key.split("/")[0] for key in z.files})


@pytest.mark.parametrize("name", golden_cases())
def test_harness_on_golden_fixtures(tmp_path, name):
    z = np.load(GOLDEN)
    q, k, v = (z[f"{name}/{x}"] for x in ("q", "k", "v"))
    print(f"case: golden {name} {q.shape} x {k.shape}", flush=True)
    o, t = run_harness(tmp_path, q, k, v, float(z[f"{name}/scale"]), reps=3)
    mx, mn = error_stats(o.astype(np.float64), z[f"{name}/o"])
    print(f"  max-abs {mx:.3e} mean-abs {mn:.3e}, {t['ms_avg']:.4f} ms", flush=True)
    assert mx <= MAX_ABS_TOL and mn <= MEAN_ABS_TOL


def test_harness_vae_head_split(tmp_path):
    B, H, S, D = 1, 1, 4096, 512
    print(f"case: VAE head B{B} H{H} S{S} D{D}", flush=True)
    qc, kc, vc = make_inputs(B, H, S, S, D, seed=8)
    o, t = run_harness(tmp_path, qc.numpy(), kc.numpy(), vc.numpy(), D ** -0.5, reps=20)
    rows = torch.arange(0, S, 32)
    ref = sdpa_math_fp32(qc[:, :, rows], kc, vc, D ** -0.5)
    mx, mn = error_stats(o[:, :, rows.numpy()].astype(np.float64), ref)
    print(f"  max-abs {mx:.3e} mean-abs {mn:.3e}; launch() {t['ms_avg']:.4f} ms avg, "
          f"{t['ms_min']:.4f} ms min, {t['tflops']} TFLOP/s", flush=True)
    assert mx <= MAX_ABS_TOL and mn <= MEAN_ABS_TOL
