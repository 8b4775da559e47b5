"""GPU parity of the gfx950 attention forward against the CPU oracle.

Every comparison uses the north-star bar: max-abs <= 2e-3 and mean-abs <= 2e-4
against torch SDPA MATH in fp32 on the same fp16 inputs (oracle.attention).
Inputs are drawn on the CPU from a seeded generator, so the oracle and the GPU
see identical bits. Shapes follow the reference's own GPU checks (test.py:23-27,
test_variants.py:78-81, test_d512.py:8-20) and BASELINE.json's five configs;
for configs whose full CPU reference would take too long, seeded query-row
slices are checked against the full K/V (the reference does the same for long
S, test.py:14-18) and the whole output is checked against a float64 torch
reference computed on the GPU, plus size-independent properties.
"""

import os

import numpy as np
import pytest
import torch

import gfx906_amd
from oracle.attention import (CONFIGS, MAX_ABS_TOL, MEAN_ABS_TOL, config_inputs, error_stats,
                              within_tolerance,
                              make_inputs, sdpa_math_fp32)

pytestmark = pytest.mark.gpu

DEV = "cuda"


def run_capi(q, k, v, scale):
    """One call through the C ABI (launch-equivalent attn_fwd) on the current stream."""
    lib = gfx906_amd.capi()
    B, H, Sq, D = q.shape
    Skv = k.shape[2]
    o = torch.empty_like(q)
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.attn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H, Sq, Skv, D,
                      float(scale), stream)
    assert rc == 0, lib.attn_last_error()
    torch.cuda.synchronize()
    return o


def run_launch(q, k, v, scale):
    """One call through the reference-compatible void launch()."""
    lib = gfx906_amd.capi()
    B, H, Sq, D = q.shape
    o = torch.empty_like(q)
    lib.launch(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H, Sq, k.shape[2], D,
               float(scale), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert lib.attn_last_error() is None
    return o


def gpu_fp64_reference(q, k, v, scale, rows=4096):
    """float64 softmax(scale q k^T) v on the GPU, per head and row block: exact
    to ~1e-15 on the fp16 inputs, so the whole-output checks do not depend on
    how the GPU's float32 GEMMs round (SDPA MATH in float32, the bar's
    reference, is within 5e-6 of it on every config)."""
    B, H, Sq, D = q.shape
    out = torch.empty(q.shape, dtype=torch.float64, device=q.device)
    for b in range(B):
        for h in range(H):
            kf = k[b, h].double()
            vf = v[b, h].double()
            for r0 in range(0, Sq, rows):
                s = (q[b, h, r0:r0 + rows].double() @ kf.t()) * scale
                out[b, h, r0:r0 + rows] = torch.softmax(s, dim=-1) @ vf
    return out


def assert_close(out, ref, what):
    mx, mn = error_stats(out.float().cpu(), ref)
    print(f"{what}: max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)
    assert mx <= MAX_ABS_TOL and mn <= MEAN_ABS_TOL, (what, mx, mn)


def check_full(B, H, Sq, Skv, D, scale=None, seed=0, qk_mult=1.0, v_mult=1.0, via="capi"):
    q, k, v = make_inputs(B, H, Sq, Skv, D, qk_mult, v_mult, seed)
    scale = D ** -0.5 if scale is None else scale
    fn = run_capi if via == "capi" else (lambda *a: gfx906_amd.attn(*a))
    out = fn(q.to(DEV), k.to(DEV), v.to(DEV), scale)
    torch.cuda.synchronize()
    ref = sdpa_math_fp32(q, k, v, scale)
    assert_close(out, ref, f"B{B} H{H} Sq{Sq} Skv{Skv} D{D} scale{scale:.4g}")
    return out


# -- reference harness shapes -------------------------------------------------

@pytest.mark.parametrize("S", [64, 256, 1024, 4096, 100, 1000])
def test_reference_test_py_d64(S):
    # test.py:23-24: B=2, H=8, D=64, scale 0.125
    check_full(2, 8, S, S, 64, scale=0.125, seed=S)


@pytest.mark.parametrize("D", [32, 16])
def test_reference_test_py_small_d(D):
    # test.py:26-27: generic head dims
    check_full(2, 8, 512, 512, D, scale=0.125, seed=D)


@pytest.mark.parametrize("Sq,Skv,D", [(256, 256, 64), (1024, 1024, 64), (100, 300, 64),
                                      (256, 256, 128), (1024, 1024, 128), (77, 411, 128),
                                      (512, 512, 32), (512, 512, 512)])
def test_reference_variant_shapes(Sq, Skv, D):
    # test_variants.py:78-81: B=2, H=4, scale 0.125
    check_full(2, 4, Sq, Skv, D, scale=0.125, seed=Sq * 7 + Skv + D)


@pytest.mark.parametrize("D", [8, 24, 40, 48, 56])
def test_generic_head_dims(D):
    check_full(1, 3, 333, 257, D, seed=D)


@pytest.mark.parametrize("S", [256, 1024, 4096])
def test_reference_d512_shapes(S):
    # test_d512.py:8-20: one head, D=512, scale c**-0.5
    check_full(1, 1, S, S, 512, seed=S)


# -- BASELINE.json configs ----------------------------------------------------

def test_config_c1_full():
    B, H, Sq, Skv, D, *_ = CONFIGS["c1"]
    q, k, v = config_inputs("c1")
    out = run_capi(q.to(DEV), k.to(DEV), v.to(DEV), D ** -0.5)
    assert_close(out, sdpa_math_fp32(q, k, v, D ** -0.5), "c1")


def _slice_rows(Sq, n, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randperm(Sq, generator=g)[:n].sort().values


@pytest.mark.parametrize("name,nrows", [("c2", 512), ("c3", 512), ("c4", 256), ("c5", 256),
                                        ("ns", 256)])
def test_config_row_slice_vs_oracle(name, nrows):
    """Seeded query-row slice of every head against the CPU oracle on full K/V."""
    B, H, Sq, Skv, D, *_ = CONFIGS[name]
    q, k, v = config_inputs(name)
    scale = D ** -0.5
    out = run_capi(q.to(DEV), k.to(DEV), v.to(DEV), scale).cpu()
    rows = _slice_rows(Sq, nrows, seed=sum(map(ord, name)))
    ref = sdpa_math_fp32(q[:, :, rows], k, v, scale)
    assert_close(out[:, :, rows], ref, f"{name} slice of {nrows} rows")
    # Whole output: finite, and inside the per-dim range of V (a convex combination).
    assert torch.isfinite(out.float()).all()
    vmin = v.float().amin(dim=2, keepdim=True)
    vmax = v.float().amax(dim=2, keepdim=True)
    slack = 1e-3 * (1 + torch.maximum(vmax.abs(), vmin.abs()))
    assert (out.float() >= vmin - slack).all() and (out.float() <= vmax + slack).all()


@pytest.mark.parametrize("name", ["c2", "c3", "c4", "c5", "ns"])
def test_config_full_vs_gpu_fp64(name):
    """Whole output against a float64 torch reference on the GPU, at the
    north-star bar for every element (max-abs <= 2e-3, mean-abs <= 2e-4).

    c3 (q, k ~ 2 N(0,1)) is the binding case: its sharp rows reach |o| > 4,
    where fp16 output rounding alone takes up to 1.95e-3 of the budget.
    """
    B, H, Sq, Skv, D, *_ = CONFIGS[name]
    q, k, v = (t.to(DEV) for t in config_inputs(name))
    scale = D ** -0.5
    out = run_capi(q, k, v, scale)
    ref = gpu_fp64_reference(q, k, v, scale)
    d = (out.double() - ref).abs()
    mx, mn = d.max().item(), d.mean().item()
    over = int((d > MAX_ABS_TOL).sum().item())
    # The floor: the exact result rounded to fp16 (RNE), as any fp16-output
    # kernel must round it.
    floor = (ref.to(q.dtype).double() - ref).abs().max().item()
    print(f"{name} full vs GPU fp64: max-abs {mx:.3e} mean-abs {mn:.3e}, "
          f"{over} elements above {MAX_ABS_TOL}; correctly rounded output {floor:.3e}",
          flush=True)
    assert mx <= MAX_ABS_TOL and mn <= MEAN_ABS_TOL, (name, mx, mn)


def _golden_cases():
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "attn_golden.npz")
    with np.load(path) as z:
        names = sorted({f.split("/")[0] for f in z.files})
        return [(n, {key: z[f"{n}/{key}"] for key in ("q", "k", "v", "o", "scale")})
                for n in names]


@pytest.mark.parametrize("name,case", _golden_cases(), ids=lambda x: x if isinstance(x, str) else "")
def test_golden_fixtures(name, case):
    """The committed fixtures (tests/golden/make_golden.py: fp16 inputs and
    their float64 outputs) through the C ABI and the torch op."""
    q, k, v = (torch.from_numpy(case[key]) for key in ("q", "k", "v"))
    scale = float(case["scale"])
    ref = torch.from_numpy(case["o"])
    a = run_capi(q.to(DEV), k.to(DEV), v.to(DEV), scale)
    assert_close(a, ref, f"golden {name} (C ABI)")
    b = gfx906_amd.attn(q.to(DEV), k.to(DEV), v.to(DEV), scale)
    torch.cuda.synchronize()
    assert_close(b, ref, f"golden {name} (op)")


# -- edge cases ----------------------------------------------------------------

def test_single_key_returns_v0():
    q, k, v = make_inputs(2, 3, 77, 1, 128, seed=5)
    out = run_capi(q.to(DEV), k.to(DEV), v.to(DEV), 0.1).cpu()
    assert torch.equal(out, v.expand_as(out))


def test_empty_keys_returns_zeros():
    q, k, v = make_inputs(1, 2, 50, 0, 64, seed=6)
    o = torch.full_like(q, float("nan")).to(DEV)
    lib = gfx906_amd.capi()
    rc = lib.attn_fwd(q.to(DEV).data_ptr(), 0, 0, o.data_ptr(), 1, 2, 50, 0, 64, 0.125,
                      torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0
    assert torch.equal(o.cpu(), torch.zeros_like(q))


@pytest.mark.parametrize("Sq", [1, 31, 33, 129])
def test_ragged_query_counts(Sq):
    check_full(1, 2, Sq, 200, 128, seed=Sq)
    check_full(1, 2, Sq, 65, 64, seed=Sq + 1)


@pytest.mark.parametrize("Skv", [1, 2, 31, 63, 65, 127, 129])
def test_ragged_key_counts(Skv):
    check_full(1, 2, 96, Skv, 128, seed=Skv)
    check_full(1, 2, 96, Skv, 64, seed=Skv + 1)
    check_full(1, 1, 40, Skv, 512, seed=Skv + 2)


def test_zero_scale_is_mean_of_v():
    q, k, v = make_inputs(1, 2, 64, 300, 64, seed=9)
    out = run_capi(q.to(DEV), k.to(DEV), v.to(DEV), 0.0).cpu().float()
    ref = v.double().mean(dim=2, keepdim=True).expand_as(out)
    assert_close(out, ref, "scale 0")


@pytest.mark.parametrize("D", [64, 128, 512])
def test_negative_scale(D):
    check_full(1, 2, 100, 300, D, scale=-(D ** -0.5), seed=11)


def test_sharp_softmax_c3_like():
    check_full(1, 2, 256, 512, 64, qk_mult=2.0, seed=12)


@pytest.mark.parametrize("nsplit", [2, 5])
@pytest.mark.parametrize("D", [40, 64, 128, 512])
def test_semantics_with_forced_splits(monkeypatch, D, nsplit):
    # The edge cases above again with the key range split (the attn_fwd entry
    # point, static scratch; GFX906_AMD_ATTN_NSPLIT forces the count): a
    # negative and a zero scale, sharp rows, a single key, and a score step
    # that the running max of one split never sees.
    monkeypatch.setenv("GFX906_AMD_ATTN_NSPLIT", str(nsplit))
    check_full(1, 2, 100, 700, D, scale=-(D ** -0.5), seed=40 + D)
    q, k, v = make_inputs(1, 2, 64, 700, D, seed=41 + D)
    out = run_capi(q.to(DEV), k.to(DEV), v.to(DEV), 0.0).cpu().float()
    assert_close(out, v.double().mean(dim=2, keepdim=True).expand_as(out), f"scale 0 D{D}")
    check_full(1, 2, 256, 700, D, qk_mult=2.0, seed=42 + D)
    q, k, v = make_inputs(1, 2, 33, 1, D, seed=43 + D)
    out = run_capi(q.to(DEV), k.to(DEV), v.to(DEV), 0.1).cpu()
    assert torch.equal(out, v.expand_as(out))
    q, k, v = make_inputs(1, 2, 96, 700, D, seed=44 + D)
    q = torch.ones_like(q) * 0.25
    k = torch.zeros_like(k)
    scale = D ** -0.5
    k[:, :, 400:, :] = 17.0 / (D * 0.25 * scale * 1.4426950408889634)
    out = run_capi(q.to(DEV), k.to(DEV), v.to(DEV), scale)
    assert_close(out, sdpa_math_fp32(q, k, v, scale), f"score step, {nsplit} splits, D{D}")


def test_large_scores_rescale():
    # Scores growing along the key axis force repeated running-max updates.
    q, k, v = make_inputs(1, 1, 64, 1024, 128, seed=13)
    ramp = torch.linspace(0.1, 4.0, 1024).view(1, 1, 1024, 1)
    k = (k.float() * ramp).half()
    out = run_capi(q.to(DEV), k.to(DEV), v.to(DEV), 128 ** -0.5)
    assert_close(out, sdpa_math_fp32(q, k, v, 128 ** -0.5), "ramped keys")


@pytest.mark.parametrize("Skv", [192, 255, 256, 257, 319, 448, 511, 513, 577, 1025])
def test_tile_ring_boundaries(Skv):
    # Key tiles are 64 keys in groups of four ring stages; key counts around
    # 256-key group edges leave 0..3 padding tiles and partial last tiles.
    check_full(1, 2, 300, Skv, 128, seed=Skv + 30)
    check_full(1, 2, 257, Skv, 64, seed=Skv + 31)
    check_full(1, 1, 77, Skv, 40, seed=Skv + 32)


def run_capi_ex(q, k, v, scale):
    """One unsplit call through attn_fwd_ex (contiguous fp16 or bf16)."""
    lib = gfx906_amd.capi()
    B, H, Sq, D = q.shape
    o = torch.empty_like(q)
    dt = 1 if q.dtype == torch.bfloat16 else 0
    rc = lib.attn_fwd_ex(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H, Sq,
                         k.shape[2], D, float(scale), torch.cuda.current_stream().cuda_stream, dt,
                         None, None, None, None)
    assert rc == 0, lib.attn_last_error()
    torch.cuda.synchronize()
    return o


# Jumps (log2 units) on both sides of each kernel's rescale limit: D <= 64
# keeps the exact running max (every rise rescales), D = 128 rescales once
# some p exceeds 2^15, D = 512 once some p exceeds 2^8.
_STEP_CASES = ([(64, j) for j in (0.5, 3.0, 14.0, 17.0)]
               + [(128, j) for j in (5.0, 14.0, 14.9, 15.1, 17.0, 24.0)]
               + [(512, j) for j in (5.0, 7.9, 8.1, 12.0, 24.0)])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("D,jump", _STEP_CASES)
def test_score_step_between_blocks(D, jump, dtype):
    # Keys 400.. score `jump` log2 units above keys 0..399 for every query, so
    # the blocks after key 400 either run on the stale running max (p up to
    # 2^jump) or take the exact-max rescale, depending on the kernel's limit.
    q, k, v = make_inputs(1, 2, 96, 700, D, seed=int(jump * 10) + D)
    q = torch.ones_like(q) * 0.25
    k = torch.zeros_like(k)
    scale = D ** -0.5
    # s * scale * log2(e) = jump for the second group of keys, 0 for the first
    k[:, :, 400:, :] = jump / (D * 0.25 * scale * 1.4426950408889634)
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    out = run_capi_ex(q.to(DEV), k.to(DEV), v.to(DEV), scale)
    ref = sdpa_math_fp32(q, k, v, scale)
    mx, mn = error_stats(out.float().cpu(), ref)
    what = f"score step {jump} D{D} {dtype}"
    print(f"{what}: max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)
    f = 8 if dtype == torch.bfloat16 else 1  # bf16: 8 significand bits to fp16's 11
    assert mx <= f * MAX_ABS_TOL and mn <= f * MEAN_ABS_TOL, (what, mx, mn)


def test_many_batch_heads():
    # B*H above 65535: one workgroup per (batch, head, query tile) in grid.x,
    # with no limit on B*H other than HIP's grid size.
    check_full(65536, 1, 8, 8, 8, seed=21)
    check_full(2, 40000, 3, 5, 64, seed=22)


def test_deterministic():
    q, k, v = (t.to(DEV) for t in make_inputs(1, 4, 1000, 1000, 128, seed=14))
    a = run_capi(q, k, v, 0.1)
    b = run_capi(q, k, v, 0.1)
    assert torch.equal(a, b)


def test_key_permutation_invariance():
    q, k, v = make_inputs(1, 2, 128, 640, 128, seed=15)
    perm = torch.randperm(640, generator=torch.Generator().manual_seed(1))
    a = run_capi(q.to(DEV), k.to(DEV), v.to(DEV), 0.09).float()
    b = run_capi(q.to(DEV), k[:, :, perm].contiguous().to(DEV), v[:, :, perm].contiguous().to(DEV),
                 0.09).float()
    assert (a - b).abs().max().item() <= 2e-3


# -- boundary: torch binding and launch() ------------------------------------------

def test_torch_binding_matches_capi():
    q, k, v = (t.to(DEV) for t in make_inputs(2, 3, 300, 200, 128, seed=16))
    a = gfx906_amd.attn(q, k, v, 0.1)
    torch.cuda.synchronize()
    b = run_capi(q, k, v, 0.1)
    c = run_launch(q, k, v, 0.1)
    assert torch.equal(a, b) and torch.equal(b, c)


def test_torch_binding_non_contiguous_inputs():
    # VAE-style [b, c, h*w] -> [b, 1, h*w, c] transposed views (test_d512.py:22-30).
    g = torch.Generator().manual_seed(17)
    x = (torch.randn(1, 512, 300, generator=g) * 0.5).half()
    q = x.transpose(1, 2).unsqueeze(1)
    assert not q.is_contiguous()
    out = gfx906_amd.attn(q.to(DEV), q.to(DEV), q.to(DEV), 512 ** -0.5)
    assert_close(out, sdpa_math_fp32(q, q, q, 512 ** -0.5), "non-contiguous D=512")


def test_torch_binding_rejects():
    q = torch.zeros(1, 1, 8, 64, dtype=torch.float16, device=DEV)
    with pytest.raises(RuntimeError):
        gfx906_amd.attn(q.float(), q, q, 0.1)           # dtype
    with pytest.raises(RuntimeError):
        gfx906_amd.attn(q, q.float(), q, 0.1)           # k dtype
    with pytest.raises(RuntimeError):
        gfx906_amd.attn(q, q[:, :, :, :32], q, 0.1)     # D mismatch
    with pytest.raises(RuntimeError):
        z = torch.zeros(1, 1, 8, 100, dtype=torch.float16, device=DEV)
        gfx906_amd.attn(z, z, z, 0.1)                   # unsupported D
    with pytest.raises(RuntimeError):
        gfx906_amd.attn(q.cpu(), q.cpu(), q.cpu(), 0.1)  # not on the GPU


def test_runs_on_current_stream():
    q, k, v = (t.to(DEV) for t in make_inputs(1, 2, 512, 512, 64, seed=18))
    s = torch.cuda.Stream()
    ref = gfx906_amd.attn(q, k, v, 0.125)
    with torch.cuda.stream(s):
        out = gfx906_amd.attn(q, k, v, 0.125)
    s.synchronize()
    assert torch.equal(out, ref)


@pytest.mark.parametrize("D,Skv", [(64, 1500), (128, 1500), (128, 300), (64, 300)])
@pytest.mark.parametrize("Sq,scale_sign,q_layout", [(300, 1, "contig"), (1000, -1, "bshd"),
                                                    (257, 1, "bshd"), (33, -1, "contig")])
def test_long_key_range_q_through_lds(D, Skv, Sq, scale_sign, q_layout):
    """More than 1024 keys (D <= 64) or 256 keys (D = 128): Q goes through LDS
    as K-shaped tiles (rows past Sq load zeros, the sign of a negative scale
    applied after the read, any q sequence stride up to 2^24); D = 64 with 300
    keys takes the gathered global loads, for comparison."""
    B, H = 1, 3
    q, k, v = make_inputs(B, H, Sq, Skv, D, seed=D + Sq)
    scale = scale_sign * D ** -0.5
    if q_layout == "bshd":
        qd = torch.empty((B, Sq, H, D), dtype=q.dtype, device=DEV).transpose(1, 2)
        qd.copy_(q.to(DEV))
    else:
        qd = q.to(DEV)
    out = gfx906_amd.attn(qd, k.to(DEV), v.to(DEV), scale)
    torch.cuda.synchronize()
    ok, mx, mn = within_tolerance(out.float().cpu(), sdpa_math_fp32(q, k, v, scale))
    print(f"D{D} Sq{Sq} {q_layout} sign{scale_sign}: max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)
    assert ok, (mx, mn)
