"""Grids of several rounds, where the D = 128 ring kernel and the D <= 64 one
with the tile max prefetch into L2 the Q tile of the workgroup that starts
after them (workgroup blockIdx + CUs x workgroups per CU): the prefetch must
change nothing. Ragged Sq puts a partial query tile behind some prefetches,
[B, S, H, D] views give them a head-interleaved sequence stride, and bf16 runs
the same path; the grids' last rounds issue the empty-range form. Outputs are
compared bit for bit with contiguous fp16/bf16 calls of the same values and
against a float64 reference at the north-star bar (bf16: eight times it).
"""

import pytest
import torch

import gfx906_amd
from oracle.attention import MAX_ABS_TOL, MEAN_ABS_TOL, make_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda"


def fp64_reference(q, k, v, scale, rows=4096):
    B, H, Sq, D = q.shape
    out = torch.empty(q.shape, dtype=torch.float64, device=q.device)
    for b in range(B):
        for h in range(H):
            kf, vf = k[b, h].double(), v[b, h].double()
            for r0 in range(0, Sq, rows):
                s = (q[b, h, r0:r0 + rows].double() @ kf.t()) * scale
                out[b, h, r0:r0 + rows] = torch.softmax(s, dim=-1) @ vf
    return out


def bshd(t):
    """The same values as a [B, H, S, D] view of a [B, S, H, D] buffer."""
    B, H, S, D = t.shape
    buf = torch.empty((B, S, H, D), dtype=t.dtype, device=t.device)
    view = buf.transpose(1, 2)
    view.copy_(t)
    return view


# (B, H, Sq, Skv, D): grids of 2 * 16 * ceil(Sq / 256) workgroups, several
# rounds of 256 (D = 128) or 512 (D = 64) resident workgroups on 256 CUs;
# Skv <= 8192 keeps the D = 64 kernel on its tile-max form.
CASES = [(2, 16, 8292, 2048, 128), (2, 16, 8292, 1000, 64), (1, 24, 16100, 512, 64)]


@pytest.mark.parametrize("B,H,Sq,Skv,D", CASES)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_multi_round_grids_with_prefetch(B, H, Sq, Skv, D, dtype):
    print(f"case: B{B} H{H} Sq{Sq} Skv{Skv} D{D} {dtype}", flush=True)
    q, k, v = (t.to(DEV, dtype) for t in make_inputs(B, H, Sq, Skv, D, 1.0, 1.0, seed=77))
    scale = D ** -0.5
    ext = gfx906_amd.extension()
    out = ext.attn(q, k, v, scale)
    # strided views of the same values: bit-equal
    out_s = ext.attn(bshd(q), bshd(k), bshd(v), scale)
    assert torch.equal(out_s, out)
    # the same call again: deterministic
    assert torch.equal(ext.attn(q, k, v, scale), out)
    ref = fp64_reference(q, k, v, scale)
    d = (out.double() - ref).abs()
    mx, mn = d.max().item(), d.mean().item()
    print(f"  max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)
    mult = 8 if dtype == torch.bfloat16 else 1
    assert mx <= mult * MAX_ABS_TOL and mn <= mult * MEAN_ABS_TOL
