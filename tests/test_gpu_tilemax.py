"""The two running-max policies of the D <= 64 ring kernel (attn_fwd_pipe's
TILEMAX template flag): the max raised once per 64-key tile over both of its
blocks (chosen for up to 8192 keys per workgroup) or once per 32-key block
(longer key ranges). GFX906_AMD_ATTN_TILEMAX=0/1 forces either. Both must meet
the north-star bar against SDPA MATH on sharp inputs (q, k x 2, the c3
multiplier) at key counts around the tile edges, where the tile's second
block is partly or wholly masked, for the padded head dims too, split and
unsplit; and the default must pick the tile max for short key ranges."""

import os

import pytest
import torch

import gfx906_amd
from oracle.attention import MAX_ABS_TOL, MEAN_ABS_TOL, error_stats, make_inputs, sdpa_math_fp32

pytestmark = pytest.mark.gpu

CASES = [
    # B, H, Sq, Skv, D
    (1, 4, 700, 33, 64),
    (1, 4, 700, 64, 64),
    (2, 3, 513, 100, 64),
    (1, 8, 1024, 512, 64),
    (1, 2, 300, 1000, 40),
    (2, 2, 600, 2500, 64),
    (1, 1, 2048, 4200, 24),
]


def _run(q, k, v, scale, tilemax, split):
    old = os.environ.get("GFX906_AMD_ATTN_TILEMAX")
    os.environ["GFX906_AMD_ATTN_TILEMAX"] = tilemax
    try:
        lib = gfx906_amd.capi()
        B, H, Sq, D = q.shape
        Skv = k.shape[2]
        o = torch.full_like(q, float("nan"))
        stream = torch.cuda.current_stream().cuda_stream
        if split:
            need = lib.attn_split_workspace_bytes(B, H, Sq, Skv, D)
            ws = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
            rc = lib.attn_fwd_split(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H,
                                    Sq, Skv, D, scale, stream, 0, None, None, None, None,
                                    ws.data_ptr(), need)
        else:
            rc = lib.attn_fwd_ex(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H, Sq,
                                 Skv, D, scale, stream, 0, None, None, None, None)
        assert rc == 0, lib.attn_last_error()
        torch.cuda.synchronize()
        return o
    finally:
        if old is None:
            del os.environ["GFX906_AMD_ATTN_TILEMAX"]
        else:
            os.environ["GFX906_AMD_ATTN_TILEMAX"] = old


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_both_max_policies_meet_the_bar(case, split):
    B, H, Sq, Skv, D = case
    print(f"case: B{B} H{H} Sq{Sq} Skv{Skv} D{D} split={split}", flush=True)
    qc, kc, vc = make_inputs(B, H, Sq, Skv, D, 2.0, 1.0, seed=Skv + D)
    q, k, v = qc.cuda(), kc.cuda(), vc.cuda()
    scale = D ** -0.5
    ref = sdpa_math_fp32(qc, kc, vc, scale)
    outs = {}
    for tm in ("0", "1"):
        outs[tm] = _run(q, k, v, scale, tm, split)
        mx, mn = error_stats(outs[tm].float().cpu(), ref)
        print(f"  TILEMAX={tm}: max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)
        assert mx <= MAX_ABS_TOL and mn <= MEAN_ABS_TOL, (tm, mx, mn)


def test_default_uses_tile_max_for_short_key_ranges():
    # c3's shape (512 keys): the default equals the forced tile max bit for
    # bit; 16384 keys: the forced per-block max.
    for Skv, want in ((512, "1"), (16384, "0")):
        print(f"case: default policy Skv={Skv}", flush=True)
        q, k, v = (t.cuda() for t in make_inputs(1, 8, 2048, Skv, 64, 2.0, 1.0, seed=5))
        lib = gfx906_amd.capi()
        o = torch.empty_like(q)
        assert lib.attn_fwd_ex(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), 1, 8, 2048,
                               Skv, 64, 0.125, torch.cuda.current_stream().cuda_stream, 0,
                               None, None, None, None) == 0
        torch.cuda.synchronize()
        assert torch.equal(o, _run(q, k, v, 0.125, want, False))
