"""attn_fwd_split_static (split key ranges, workspace in the library's static
device scratch) against attn_fwd_split with a caller workspace, through the
C ABI, on two calls in a row (the second smaller, so it runs on what the first
left in the scratch). Both run the same split plan and kernels, so the
outputs must be bit-identical; both are also held to the north-star bar
against the CPU oracle."""

import ctypes

import pytest
import torch

import gfx906_amd
from oracle.attention import MAX_ABS_TOL, MEAN_ABS_TOL, error_stats, make_inputs, sdpa_math_fp32

pytestmark = pytest.mark.gpu


def _split(lib, q, k, v, scale):
    B, H, Sq, D = q.shape
    Skv = k.shape[2]
    need = lib.attn_split_workspace_bytes(B, H, Sq, Skv, D)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    o = torch.empty_like(q)
    rc = lib.attn_fwd_split(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H, Sq,
                            Skv, D, scale, torch.cuda.current_stream().cuda_stream, 0,
                            None, None, None, None, ctypes.c_void_p(ws.data_ptr()), need)
    assert rc == 0, lib.attn_last_error()
    return o, need


def _static(lib, q, k, v, scale):
    B, H, Sq, D = q.shape
    o = torch.full_like(q, float("nan"))
    rc = lib.attn_fwd_split_static(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H,
                                   Sq, k.shape[2], D, scale,
                                   torch.cuda.current_stream().cuda_stream, 0,
                                   None, None, None, None)
    assert rc == 0, lib.attn_last_error()
    return o


@pytest.mark.parametrize("first,second", [
    ((1, 1, 4096, 4096, 512), (1, 1, 1000, 1500, 512)),  # one VAE head, then a smaller one
    ((1, 4, 2048, 3000, 128), (1, 2, 700, 900, 128)),
    ((2, 2, 1024, 2048, 64), (1, 1, 300, 1111, 40)),
])
def test_static_scratch_matches_caller_workspace(first, second):
    lib = gfx906_amd.capi()
    for n, (B, H, Sq, Skv, D) in enumerate((first, second)):
        print(f"case: call {n + 1} B{B} H{H} Sq{Sq} Skv{Skv} D{D}", flush=True)
        qc, kc, vc = make_inputs(B, H, Sq, Skv, D, seed=1000 * n + D + Sq)
        q, k, v = qc.cuda(), kc.cuda(), vc.cuda()
        scale = D ** -0.5
        a, need = _split(lib, q, k, v, scale)
        assert 0 < need <= lib.attn_split_scratch_capacity()  # the call really splits
        b = _static(lib, q, k, v, scale)
        torch.cuda.synchronize()
        assert torch.equal(a, b)
        rows = torch.arange(0, Sq, max(1, Sq // 128))
        ref = sdpa_math_fp32(qc[:, :, rows], kc, vc, scale)
        mx, mn = error_stats(b[:, :, rows].float().cpu(), ref)
        print(f"  static vs oracle: max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)
        assert mx <= MAX_ABS_TOL and mn <= MEAN_ABS_TOL
