"""Split key ranges (attn_fwd_split and the torch op): problems whose
workgroups leave CUs idle are split over the keys and merged. The split
result agrees with the unsplit kernel (attn_fwd_ex) to fp32 rounding of the
merge and with SDPA MATH fp32 at the north-star bar."""

import ctypes

import pytest
import torch

import gfx906_amd
from oracle.attention import make_inputs, sdpa_math_fp32, within_tolerance

pytestmark = pytest.mark.gpu

DEV = "cuda"
F16, BF16 = 0, 1


def call(fn, q, k, v, o, scale, dtype, strides=None, ws=None):
    lib = gfx906_amd.capi()
    B, H, Sq, D = q.shape
    arrs = [None if not strides or n not in strides else (ctypes.c_longlong * 4)(*strides[n])
            for n in "qkvo"]
    args = [q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H, Sq, k.shape[2], D,
            float(scale), torch.cuda.current_stream().cuda_stream, dtype, *arrs]
    if fn == "split":
        args += [ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0]
        rc = lib.attn_fwd_split(*args)
    else:
        rc = lib.attn_fwd_ex(*args)
    torch.cuda.synchronize()
    assert rc == 0, lib.attn_last_error()


def workspace(B, H, Sq, Skv, D):
    n = gfx906_amd.capi().attn_split_workspace_bytes(B, H, Sq, Skv, D)
    return n, (torch.empty(n, dtype=torch.uint8, device=DEV) if n else None)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,H,Sq,Skv,D", [
    (1, 1, 300, 3000, 128),   # ragged Sq, last split partial
    (1, 2, 256, 4096, 64),
    (1, 1, 77, 2111, 40),     # padded head dim
    (1, 1, 1000, 2048, 512),
    (2, 1, 130, 1300, 512),
    (1, 1, 1024, 1024, 64),   # c1
])
def test_split_matches_unsplit_and_sdpa(dtype, B, H, Sq, Skv, D):
    q, k, v = (t.to(dtype).to(DEV) for t in make_inputs(B, H, Sq, Skv, D, 1.0, 1.0, Sq + Skv + D))
    n, ws = workspace(B, H, Sq, Skv, D)
    assert n > 0, "shape chosen to split"
    ref = torch.empty_like(q)
    call("ex", q, k, v, ref, D ** -0.5, F16 if dtype == torch.float16 else BF16)
    o = torch.full_like(q, float("nan"))
    call("split", q, k, v, o, D ** -0.5, F16 if dtype == torch.float16 else BF16, ws=ws)
    d = (o.float() - ref.float()).abs().max().item()
    print(f"split {dtype} B{B} H{H} Sq{Sq} Skv{Skv} D{D}: vs unsplit {d:.2e}", flush=True)
    assert d <= (2e-3 if dtype == torch.float16 else 1.6e-2)
    if dtype == torch.float16:
        exact = sdpa_math_fp32(q.float().cpu(), k.float().cpu(), v.float().cpu(), D ** -0.5)
        ok, mx, mn = within_tolerance(o.float().cpu(), exact)
        assert ok, (mx, mn)


@pytest.mark.parametrize("D,Sq,Skv", [(64, 700, 2200), (128, 300, 2500), (512, 200, 1500)])
def test_every_split_count_matches_unsplit_and_sdpa(monkeypatch, D, Sq, Skv):
    # Split counts forced from 2 to 17 and one range per key tile: the
    # merge's batches of four splits and its ragged last batch, and the split
    # kernels on ranges of a single (last: partial) tile.
    B, H = 1, 2
    q, k, v = (t.to(DEV) for t in make_inputs(B, H, Sq, Skv, D, 1.0, 1.0, seed=D + Sq))
    ref = torch.empty_like(q)
    call("ex", q, k, v, ref, D ** -0.5, F16)
    exact = sdpa_math_fp32(q.float().cpu(), k.float().cpu(), v.float().cpu(), D ** -0.5)
    tiles = -(-Skv // (32 if D == 512 else 64))
    counts = set()
    for n in list(range(2, 18)) + [tiles]:
        monkeypatch.setenv("GFX906_AMD_ATTN_NSPLIT", str(n))
        nbytes, ws = workspace(B, H, Sq, Skv, D)
        per = -(-tiles // n)
        ns = -(-tiles // per)
        assert nbytes == ns * B * H * Sq * (D + 2) * 4 + 16
        counts.add(ns)
        o = torch.full_like(q, float("nan"))
        call("split", q, k, v, o, D ** -0.5, F16, ws=ws)
        d = (o.float() - ref.float()).abs().max().item()
        ok, mx, mn = within_tolerance(o.float().cpu(), exact)
        print(f"D{D} n={n} -> {ns} splits: vs unsplit {d:.2e}, vs SDPA {mx:.2e} / {mn:.2e}",
              flush=True)
        assert d <= 2e-3 and ok, (n, d, mx, mn)
    assert len(counts) >= 9 and tiles in counts


def test_split_token_contiguous_d512_and_workspace_reuse():
    # VAE views through the in-place kernel, split; then a second, smaller
    # problem on the same workspace.
    g = torch.Generator().manual_seed(21)
    x = [(torch.randn(1, 512, 48, 48, generator=g) * 0.5).half().to(DEV) for _ in range(3)]
    views = [t.reshape(1, 512, -1).transpose(1, 2).unsqueeze(1) for t in x]
    Sq = views[0].shape[2]
    n, ws = workspace(1, 1, Sq, Sq, 512)
    assert n > 0
    st = lambda t: (0, 0, t.stride(2), t.stride(3))  # noqa: E731
    out = torch.empty(1, 512, 48, 48, dtype=torch.float16, device=DEV)
    ov = out.reshape(1, 512, -1).transpose(1, 2).unsqueeze(1)
    call("split", *views, ov, 512 ** -0.5, F16,
         {"q": st(views[0]), "k": st(views[1]), "v": st(views[2]), "o": st(ov)}, ws)
    ref = gfx906_amd.attn(*(t.contiguous() for t in views), 512 ** -0.5)
    assert (ov.float() - ref.float()).abs().max().item() <= 2e-3
    q, k, v = (t.to(DEV) for t in make_inputs(1, 1, 200, 2000, 128, seed=5))
    o = torch.empty_like(q)
    call("split", q, k, v, o, 0.1, F16, ws=ws)
    r2 = torch.empty_like(q)
    call("ex", q, k, v, r2, 0.1, F16)
    assert (o.float() - r2.float()).abs().max().item() <= 2e-3


def test_op_splits_small_grids():
    # The op takes the split path for a one-head VAE-sized call.
    q, k, v = (t.to(DEV) for t in make_inputs(1, 1, 4096, 4096, 512, 0.5, 1.0, seed=8))
    assert gfx906_amd.capi().attn_split_workspace_bytes(1, 1, 4096, 4096, 512) > 0
    got = gfx906_amd.attn(q, k, v, 512 ** -0.5)
    ref = torch.empty_like(q)
    call("ex", q, k, v, ref, 512 ** -0.5, F16)
    assert (got.float() - ref.float()).abs().max().item() <= 2e-3
