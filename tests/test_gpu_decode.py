"""Decode-like calls: a few query rows against a long key range.

The grid then has one workgroup per head and query tile, and the split key
range planner spreads the keys over up to hundreds of workgroups (196 splits
for one row over 100,000 keys), whose partial results attn_combine merges.
Each case runs through the torch op and is held to the north-star bar against
SDPA MATH in fp32 on the CPU; the number of splits the library planned is
asserted, so the case keeps exercising the many-split merge. Each case prints
its parameters first.
"""

import pytest
import torch

import gfx906_amd
from oracle.attention import MAX_ABS_TOL, MEAN_ABS_TOL, error_stats, make_inputs, sdpa_math_fp32

pytestmark = pytest.mark.gpu

CASES = [  # B, H, Sq, Skv, D, at least this many splits
    (1, 1, 1, 100000, 128, 100),
    (2, 3, 7, 65537, 64, 32),     # odd key count: a masked last tile in the last split
    (1, 2, 1, 50000, 512, 64),
    (1, 1, 5, 100000, 40, 100),   # padded head dim
]


@pytest.mark.parametrize("B,H,Sq,Skv,D,min_splits", CASES)
def test_decode_many_splits(B, H, Sq, Skv, D, min_splits):
    print(f"case decode: B{B} H{H} Sq{Sq} Skv{Skv} D{D}", flush=True)
    need = gfx906_amd.capi().attn_split_workspace_bytes(B, H, Sq, Skv, D)
    nsplit = (need - 16) // (B * H * Sq * (D + 2) * 4)
    assert nsplit >= min_splits, nsplit
    q, k, v = make_inputs(B, H, Sq, Skv, D, 1.0, 1.0, Skv % 1000 + D)
    scale = D ** -0.5
    out = gfx906_amd.attn(q.cuda(), k.cuda(), v.cuda(), scale).float().cpu()
    ref = sdpa_math_fp32(q, k, v, scale)
    mx, mn = error_stats(out, ref)
    print(f"  {nsplit} splits: max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)
    assert mx <= MAX_ABS_TOL and mn <= MEAN_ABS_TOL
