"""D = 512 kernels: attn_fwd_d512w (32 query rows per wave, the default for
row-contiguous K/V) against attn_fwd_d512 (16 rows per wave): both compute
every output row with the same operations in the same order, so their
outputs must be bit-identical; each case is also held to the north-star bar
against the CPU oracle. GFX906_AMD_ATTN_D512W=0 selects attn_fwd_d512 per
call."""

import ctypes
import os

import pytest
import torch

import gfx906_amd
from oracle.attention import MAX_ABS_TOL, MEAN_ABS_TOL, error_stats, make_inputs, sdpa_math_fp32

pytestmark = pytest.mark.gpu


def _st(t):
    return (ctypes.c_longlong * 4)(*t.stride())


def run(q, k, v, scale, wide, o_view=None, split=False):
    """wide: True = attn_fwd_d512w, False = attn_fwd_d512."""
    if not wide:
        os.environ["GFX906_AMD_ATTN_D512W"] = "0"
    try:
        lib = gfx906_amd.capi()
        B, H, Sq, D = q.shape
        Skv = k.shape[2]
        o = torch.full_like(q, float("nan")) if o_view is None else o_view
        dt = 1 if q.dtype == torch.bfloat16 else 0
        stream = torch.cuda.current_stream().cuda_stream
        args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H, Sq, Skv, D,
                float(scale), stream, dt, _st(q), _st(k), _st(v), _st(o))
        if split:
            n = lib.attn_split_workspace_bytes(B, H, Sq, Skv, D)
            assert n > 0, "expected a split problem"
            ws = torch.empty(n, dtype=torch.uint8, device=q.device)
            rc = lib.attn_fwd_split(*args, ws.data_ptr(), n)
        else:
            rc = lib.attn_fwd_ex(*args)
        assert rc == 0, lib.attn_last_error()
        torch.cuda.synchronize()
        return o
    finally:
        os.environ.pop("GFX906_AMD_ATTN_D512W", None)


def check(q, k, v, scale, what, rows=None, split=False):
    a = run(q, k, v, scale, wide=False, split=split)
    b = run(q, k, v, scale, wide=True, split=split)
    assert torch.equal(a, b), f"{what}: attn_fwd_d512w differs from attn_fwd_d512"
    Sq = q.shape[2]
    rows = torch.arange(Sq) if rows is None else rows
    ref = sdpa_math_fp32(q.cpu()[:, :, rows], k.cpu(), v.cpu(), scale)
    mx, mn = error_stats(b.cpu()[:, :, rows].float(), ref)
    f = 8 if q.dtype == torch.bfloat16 else 1
    print(f"{what}: max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)
    assert mx <= f * MAX_ABS_TOL and mn <= f * MEAN_ABS_TOL, (what, mx, mn)


def test_c4_bit_identical():
    print("case: c4 B1 H4 S8192 D512", flush=True)
    q, k, v = (t.cuda() for t in make_inputs(1, 4, 8192, 8192, 512, 1.0, 1.0, seed=4))
    g = torch.Generator().manual_seed(40)
    rows = torch.randperm(8192, generator=g)[:128].sort().values
    check(q, k, v, 512 ** -0.5, "c4", rows)


@pytest.mark.parametrize("Skv", [1, 31, 32, 33, 64, 95, 1000])
def test_key_counts(Skv):
    # 300 query rows: three 128-row tiles, the last ragged (44 rows: one
    # wave full, one half full, two empty).
    print(f"case: B2 H3 Sq300 Skv{Skv} D512", flush=True)
    q, k, v = (t.cuda() for t in make_inputs(2, 3, 300, Skv, 512, 2.0, 1.0, seed=Skv))
    check(q, k, v, 512 ** -0.5, f"Skv{Skv}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_strided_views_negative_scale_and_sharp_rows(dtype):
    # [B, S, H, D] buffers viewed as [B, H, S, D]; q doubled so that the
    # running max moves between tiles (rescale path) on many rows.
    B, H, Sq, Skv, D = 1, 2, 400, 700, 512
    print(f"case: strided {dtype} B{B} H{H} Sq{Sq} Skv{Skv}", flush=True)
    g = torch.Generator().manual_seed(5)
    qb = (3 * torch.randn(B, Sq, H, D, generator=g)).to("cuda", dtype)
    kb = torch.randn(B, Skv, H, D, generator=g).to("cuda", dtype)
    vb = torch.randn(B, Skv, H, D, generator=g).to("cuda", dtype)
    q, k, v = (t.transpose(1, 2) for t in (qb, kb, vb))
    outs = []
    for wide in (False, True):
        ob = torch.full((B, Sq, H, D), float("nan"), dtype=dtype, device="cuda")
        outs.append(run(q, k, v, -0.06, wide, o_view=ob.transpose(1, 2)))
    assert torch.equal(outs[0], outs[1])
    ref = sdpa_math_fp32(q.cpu(), k.cpu(), v.cpu(), -0.06)
    mx, mn = error_stats(outs[1].cpu().float(), ref)
    f = 8 if dtype == torch.bfloat16 else 1
    print(f"strided {dtype}: max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)
    assert mx <= f * MAX_ABS_TOL and mn <= f * MEAN_ABS_TOL, (mx, mn)


def test_split_key_ranges():
    # One head of 4096 tokens: 32 query tiles, split over the key range.
    print("case: split B1 H1 S4096 D512", flush=True)
    q, k, v = (t.cuda() for t in make_inputs(1, 1, 4096, 4096, 512, 1.0, 1.0, seed=7))
    g = torch.Generator().manual_seed(8)
    rows = torch.randperm(4096, generator=g)[:256].sort().values
    check(q, k, v, 512 ** -0.5, "split", rows, split=True)


def test_no_keys_gives_zeros():
    q = torch.randn(1, 2, 130, 512, device="cuda").half()
    k = torch.empty(1, 2, 0, 512, device="cuda").half()
    o = run(q, k, k, 0.1, wide=True)
    assert torch.equal(o, torch.zeros_like(o))


def test_default_dispatch_is_wide():
    # The torch op agrees with the wide kernel bit for bit on a problem that
    # fills the GPU without splitting the key range (8 x 32 query tiles).
    q, k, v = (t.cuda() for t in make_inputs(1, 8, 4096, 256, 512, 1.0, 1.0, seed=9))
    assert gfx906_amd.capi().attn_split_workspace_bytes(1, 8, 4096, 256, 512) == 0
    b = run(q, k, v, 0.05, wide=True)
    op = gfx906_amd.attn(q, k, v, 0.05)
    torch.cuda.synchronize()
    assert torch.equal(op, b)
