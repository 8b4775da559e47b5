"""NaN propagation of the gfx950 attention forward against torch SDPA MATH.

The reference kernel has no test for non-finite inputs. torch SDPA MATH (the
parity target) propagates a NaN in a query row to that output row only, a
NaN in any key row to every output row of its head (the key's score enters
every row's softmax), and a NaN in any value row to every output row of its
head (0 * NaN is NaN even where the weight underflows). The kernel's running
maximum, its rescale tests and its split-key merge (each case runs with the
op's own plan and with its keys forced into three ranges) must keep exactly
that pattern and leave every other row at the usual bar. Each case prints its
parameters first.
"""

import math

import pytest
import torch

import gfx906_amd
from oracle.attention import error_stats, make_inputs, sdpa_math_fp32, MAX_ABS_TOL, MEAN_ABS_TOL

pytestmark = pytest.mark.gpu

CASES = [  # B, H, Sq, Skv, D
    (1, 3, 300, 260, 40),
    (1, 3, 300, 260, 64),
    (2, 2, 520, 1100, 64),
    (1, 3, 300, 260, 128),
    (2, 2, 520, 1100, 128),
    (1, 2, 200, 96, 512),
]


@pytest.mark.parametrize("nsplit", [None, 3])
@pytest.mark.parametrize("B,H,Sq,Skv,D", CASES)
@pytest.mark.parametrize("where", ["q", "k", "v"])
def test_nan_pattern_matches_sdpa(monkeypatch, B, H, Sq, Skv, D, where, nsplit):
    # nsplit: the op's own plan, or the key range forced into three ranges
    # (GFX906_AMD_ATTN_NSPLIT), so that the NaN passes through the merge.
    if nsplit:
        monkeypatch.setenv("GFX906_AMD_ATTN_NSPLIT", str(nsplit))
    print(f"case nan in {where}: B{B} H{H} Sq{Sq} Skv{Skv} D{D} nsplit {nsplit}", flush=True)
    q, k, v = make_inputs(B, H, Sq, Skv, D, 1.0, 1.0, 7)
    t = {"q": q, "k": k, "v": v}[where]
    rows = t.shape[2]
    # one NaN element in head 1 of batch 0, in a row past the first tile
    t[0, 1, min(rows - 1, 70), D // 2] = float("nan")
    scale = 1.0 / math.sqrt(D)
    out = gfx906_amd.attn(q.cuda(), k.cuda(), v.cuda(), scale).float().cpu()
    torch.cuda.synchronize()
    ref = sdpa_math_fp32(q, k, v, scale)
    nan_out, nan_ref = torch.isnan(out), torch.isnan(ref)
    assert torch.equal(nan_out, nan_ref), (where, int(nan_out.sum()), int(nan_ref.sum()))
    assert nan_ref.any()
    fin = ~nan_ref
    assert torch.isfinite(out[fin]).all()
    mx, mn = error_stats(out[fin], ref[fin])
    print(f"  finite part: max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)
    assert mx <= MAX_ABS_TOL and mn <= MEAN_ABS_TOL
