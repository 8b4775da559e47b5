"""Seeded random sweep of the gfx950 conv3d over shapes, windows, strides,
bias / residual and kernel configurations, against the CPU oracle.

Each case draws (from its own seed) N, C and K (multiples of 8), the input
extent, a window of 1..3 per axis, strides of 1 or 2, bias and residual on or
off, and either the launcher's own kernel choice or one kernel forced through
GFX906_AMD_CONV_CFG, so that every configuration also meets shapes nobody
picked by hand. Bar: the conv3d parity tests' (every output within the fp16
half-ulp of the exact fp64 result plus 1e-3, and the reference's allclose
2e-2).
"""

import os

import numpy as np
import pytest
import torch

from gfx906_amd import kitchen
from oracle import conv3d as oc

pytestmark = pytest.mark.gpu

DEV = "cuda"
CL = torch.channels_last_3d
N_CASES = int(os.environ.get("GFX906_AMD_CONV_SWEEP_CASES", "32"))  # longer: same generator
CFGS = ["auto", "4x32", "3x64", "2x64", "4x32x256", "3x32x256", "3x64x256", "2x64x256"]


def draw_case(i):
    rng = np.random.default_rng(9000 + i)
    n = int(rng.integers(1, 3))
    c = 8 * int(rng.choice([1, 2, 3, 5, 8, 12, 16, 32, 64]))
    k = 8 * int(rng.choice([1, 2, 4, 7, 16, 33, 64]))
    t, r, s = (int(rng.integers(1, 4)) for _ in range(3))
    stride = tuple(int(rng.choice([1, 1, 2])) for _ in range(3))
    d = t + int(rng.integers(0, 6))
    h = r + int(rng.integers(0, 24))
    w = s + int(rng.integers(0, 24))
    cfg = str(rng.choice(CFGS))
    return dict(xs=(n, c, d, h, w), ws=(k, t, r, s), stride=stride, bias=bool(rng.random() < 0.7),
                res=bool(rng.random() < 0.4), cfg=cfg, seed=9000 + i)


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_conv3d(monkeypatch, i):
    c = draw_case(i)
    print(c, flush=True)
    if c["cfg"] == "auto":
        monkeypatch.delenv("GFX906_AMD_CONV_CFG", raising=False)
    else:
        monkeypatch.setenv("GFX906_AMD_CONV_CFG", c["cfg"])
    x, w, b, res = oc.make_case(c["xs"], c["ws"], c["stride"], c["bias"], c["res"], c["seed"])
    dev = lambda a: None if a is None else torch.from_numpy(a).to(DEV)
    xd = dev(x).contiguous(memory_format=CL)
    wd = dev(w).contiguous(memory_format=CL)
    rd = None if res is None else dev(res).contiguous(memory_format=CL)
    got = kitchen.try_kernel(xd, wd, dev(b), rd, list(c["stride"]))
    torch.cuda.synchronize()
    assert got is not None, "kernel declined"
    exact = torch.from_numpy(oc.conv3d_gemm(x, w, b, res, c["stride"]))
    g = got.float().cpu().double()
    d = (g - exact).abs()
    _, e = torch.frexp(exact.abs())
    half_ulp = torch.ldexp(torch.ones_like(exact), (e - 12).clamp(min=-25))
    print(f"case {i}: max-abs {d.max().item():.3e}", flush=True)
    assert torch.allclose(g, exact, atol=2e-2, rtol=2e-2)
    assert bool((d <= half_ulp + 1e-3).all()), d.max().item()
