"""Seeded random sweep of the C ABI entry points with explicit strides.

The torch-op sweep (test_gpu_sweep.py) reaches the kernels through the op's
own layout and split decisions. This one calls the library as a C caller
does (ctypes, element strides per tensor) and runs every case three ways:

* ``attn_fwd_ex``: one workgroup per query tile, never a split, whatever
  the grid size;
* ``attn_fwd_split`` with a caller workspace sized by
  ``attn_split_workspace_bytes`` (the key range split when the grid is small);
* ``attn_fwd_split_static``: the same split in the library's static scratch,
  which must give the same bits as the caller-workspace call.

In about half the cases the two split calls run with a forced split count (2 to 9,
GFX906_AMD_ATTN_NSPLIT), also on grids the planner would not split.

Each case draws a head dim from every class, fp16 or bf16, B and H, ragged Sq
and Skv (up to 2500 keys, so Q through LDS and several splits occur), a scale
of either sign, and a layout per tensor (contiguous, [B, S, H, D] transpose,
padded sequence stride, K/V shared by every head with head stride 0, and for
D = 512 the token-contiguous K/V of a [b, c, h*w] activation). Outputs of the
first two calls are held to the bars of the other parity tests against SDPA
MATH in fp32 on the CPU (fp16 2e-3 / 2e-4, bf16 eight times that), except
where the output format's spacing leaves no room under the bars: there an
element may be off by half a unit in the last place of the reference plus the
mean bar (fp16 from |o| >= 4, where the correctly rounded output alone errs by
up to 1.95e-3), and the mean error may reach that of the correctly rounded
reference plus half the mean bar (within_rounded_tolerance). Each case prints
its parameters first.
"""

import ctypes
import os

import numpy as np
import pytest
import torch

import gfx906_amd
from oracle.attention import make_inputs, sdpa_math_fp32, within_rounded_tolerance

pytestmark = pytest.mark.gpu

# GFX906_AMD_CAPI_SWEEP_CASES=400 runs a longer sweep (same generator, more seeds).
N_CASES = int(os.environ.get("GFX906_AMD_CAPI_SWEEP_CASES", "48"))
HEAD_DIMS = [8, 24, 40, 56, 64, 64, 128, 128, 128, 512, 512]
F16, BF16 = 0, 1


def strides(t):
    """{batch, head, seq, dim} element strides for the C ABI (0 for size-1
    batch, head and sequence dims, whose stride is never used)."""
    return (ctypes.c_longlong * 4)(*[0 if d < 3 and t.size(d) == 1 else t.stride(d)
                                     for d in range(4)])


def place(x, how, rng):
    """x [B, H, S, D] on the GPU in layout `how`, same values."""
    B, H, S, D = x.shape
    if how == "bshd":
        t = torch.empty((B, S, H, D), dtype=x.dtype, device="cuda").transpose(1, 2)
    elif how == "pad":
        pad = 8 * int(rng.integers(1, 4))
        t = torch.empty((B, H, S, D + pad), dtype=x.dtype, device="cuda")[..., :D]
    elif how == "tl":  # [B, D, S] activation seen as [B, 1, S, D]
        t = torch.empty((B, D, S), dtype=x.dtype, device="cuda").transpose(1, 2).unsqueeze(1)
    else:
        t = torch.empty((B, H, S, D), dtype=x.dtype, device="cuda")
    t.copy_(x.to("cuda"))
    return t


def draw_case(i):
    rng = np.random.default_rng(9100 + i)
    D = int(rng.choice(HEAD_DIMS))
    dtype = torch.bfloat16 if rng.random() < 0.3 else torch.float16
    B, H = int(rng.integers(1, 3)), int(rng.integers(1, 4))
    smax = 800 if D == 512 else 2500
    Sq = int(np.exp(rng.uniform(0, np.log(smax))))
    Skv = int(np.exp(rng.uniform(0, np.log(smax))))
    scale = float(rng.choice([-1, 1]) * rng.uniform(0.5, 1.0) * D ** -0.5)
    qk_mult = float(rng.choice([1.0, 1.0, 2.0]))
    lay = [str(rng.choice(["contig", "bshd", "pad"])) for _ in range(4)]
    if H > 1 and rng.random() < 0.25:
        lay[1] = lay[2] = "bcast"
    if D == 512 and rng.random() < 0.5:
        H = 1
        Skv = max(8, Skv - Skv % 8)
        lay[1] = lay[2] = "tl"
    return dict(D=D, dtype=dtype, B=B, H=H, Sq=Sq, Skv=Skv, scale=scale, qk_mult=qk_mult,
                lay=lay, seed=9100 + i), rng


@pytest.fixture(scope="module")
def lib():
    return gfx906_amd.capi()


@pytest.mark.parametrize("i", range(N_CASES))
def test_capi_random_case(lib, i, monkeypatch):
    c, rng = draw_case(i)
    # About half the cases force the split count (GFX906_AMD_ATTN_NSPLIT, 2..9) for
    # the two split calls, from a generator of its own so that the cases'
    # other draws stay as they were.
    ns = int(np.random.default_rng(1_000_000 + i).integers(0, 18))
    c["nsplit"] = ns if ns >= 2 and ns <= 9 else None
    if c["nsplit"]:
        monkeypatch.setenv("GFX906_AMD_ATTN_NSPLIT", str(c["nsplit"]))
    print(c, flush=True)
    B, H, Sq, Skv, D = c["B"], c["H"], c["Sq"], c["Skv"], c["D"]
    q, k, v = make_inputs(B, H, Sq, Skv, D, c["qk_mult"], 1.0, c["seed"])
    if c["lay"][1] == "bcast":
        k, v = k[:, :1].expand(B, H, Skv, D), v[:, :1].expand(B, H, Skv, D)
    q, k, v = (t.to(c["dtype"]) for t in (q, k, v))
    qd = place(q, c["lay"][0], rng)
    if c["lay"][1] == "bcast":
        kd = place(k[:, :1], "contig", rng).expand(B, H, Skv, D)
        vd = place(v[:, :1], "contig", rng).expand(B, H, Skv, D)
    else:
        kd, vd = place(k, c["lay"][1], rng), place(v, c["lay"][2], rng)
    dt = BF16 if c["dtype"] == torch.bfloat16 else F16
    stream = torch.cuda.current_stream().cuda_stream
    outs = [place(torch.full((B, H, Sq, D), float("nan"), dtype=c["dtype"]), c["lay"][3], rng)
            for _ in range(3)]
    args = lambda o: (qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), o.data_ptr(), B, H, Sq, Skv,
                      D, c["scale"], stream, dt, strides(qd), strides(kd), strides(vd),
                      strides(o))
    assert lib.attn_fwd_ex(*args(outs[0])) == 0, lib.attn_last_error()
    need = lib.attn_split_workspace_bytes(B, H, Sq, Skv, D)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    assert lib.attn_fwd_split(*args(outs[1]), ctypes.c_void_p(ws.data_ptr()), need) == 0, \
        lib.attn_last_error()
    static = need <= lib.attn_split_scratch_capacity()
    if static:
        assert lib.attn_fwd_split_static(*args(outs[2])) == 0, lib.attn_last_error()
    torch.cuda.synchronize()
    if static:
        assert torch.equal(outs[1], outs[2])
    ref = sdpa_math_fp32(q.contiguous(), k.contiguous(), v.contiguous(), c["scale"])
    for name, o in (("ex", outs[0]), ("split", outs[1])):
        if c["dtype"] == torch.float16:
            ok, mx, mn = within_rounded_tolerance(o.float().cpu(), ref, "fp16")
        else:
            ok, mx, mn = within_rounded_tolerance(o.float().cpu(), ref, "bf16", mult=8)
        print(f"  {name} (workspace {need} B): max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)
        assert ok, (name, c, mx, mn)
