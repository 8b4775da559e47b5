"""CPU oracle for the attention forward. TEST INFRASTRUCTURE ONLY.

Nothing in the product (``gfx906_amd``) imports this module. It is used by
``tests/``, ``__graft_entry__.smoke()`` as the checker, and ``bench.py``'s
``cpu_baseline`` leg as the timed CPU path.

Functions and what pins each one (tests/test_oracle.py):

* :func:`attention_fp64` -- direct softmax(scale*QK^T)V in float64, the
  semantics of the reference's kernels (attn_kernel.hip:313-512 pair kernel,
  :525-708 D=512 kernel, :146-308 generic kernel: scale applied to the dot,
  no mask, Sq != Skv). Pinned by closed forms (Skv=1 -> v0, q=0 -> mean(V),
  one-hot V -> the probabilities, shift/permutation invariance, scale
  folding, convex hull), by brute-force per-element loops on tiny shapes and
  by agreement with torch's SDPA MATH (a library routine) to 1e-12 in
  float64.
* :func:`sdpa_math_fp32` -- torch SDPA restricted to the MATH backend on CPU,
  on the float32 upcast of the fp16 inputs: the parity target named by the
  north star. Library routine; pinned against :func:`attention_fp64`.
* :func:`online_softmax_tiled` -- restatement of the reference's streaming
  state machine (attn_kernel.hip:357 init m=-inf, l=0; :452-462 tile max,
  exp, rescale factor rs = l>0 ? exp(m-m') : 0; :486-492 acc/l update;
  :497-511 o = acc/l only when l > 0), vectorised over rows, in float64 with
  the tile size as a parameter. Pinned against :func:`attention_fp64` for
  several tile sizes and odd Sq != Skv, the check the reference's own CPU
  model makes (model_check.py:139-153).
* :func:`kernel_numerics_model` -- the gfx950 kernel's rounding choices
  (fp32 scores and softmax state, fp16-rounded P, row sum taken from the
  rounded P, the per-head-dim rescale limit taken over the kernel's key
  tile and row group, fp16 output) in numpy. Pinned against :func:`attention_fp64` within the
  north-star tolerance, and against the one c3 element a stale running max
  moves past the bar; it documents why the kernel's numerics meet the bar,
  it is not what the GPU output is compared with.
* :func:`chunked_sdpa_math` -- :func:`sdpa_math_fp32` over head / row
  blocks, bounding memory for long sequences; pinned against the unchunked
  call.
* :func:`within_rounded_tolerance` -- the north-star bars where the output
  format's spacing allows them, else half an ulp plus the mean bar, element
  by element, and for the mean the correctly rounded reference's own mean
  error plus half the mean bar; pinned by correctly rounded fp16 and bf16
  values, the per-magnitude limits of fp16 and bf16, the seeded sweeps'
  rounding-boundary elements and outputs one ulp off.
* :func:`round_to_format` -- round to nearest even in fp16 or bf16; pinned
  against torch's own fp16 and bf16 conversions.

Skv == 0: every function returns zeros (torch SDPA MATH on CPU returns zeros
for an empty key set; the reference kernel leaves those rows unwritten).
"""

from __future__ import annotations

import math
import time

import numpy as np

LOG2E = 1.4426950408889634

# Tolerance of the north star: against SDPA MATH in fp32 on the same fp16 inputs.
MAX_ABS_TOL = 2e-3
MEAN_ABS_TOL = 2e-4


def _as64(x):
    try:
        import torch

        if isinstance(x, torch.Tensor):
            return x.detach().to("cpu", torch.float64).numpy()
    except ImportError:  # pragma: no cover
        pass
    return np.asarray(x, dtype=np.float64)


def attention_fp64(q, k, v, scale):
    """softmax(scale * q k^T) v in float64; q [..., Sq, D], k/v [..., Skv, D]."""
    q, k, v = _as64(q), _as64(k), _as64(v)
    if k.shape[-2] == 0:
        return np.zeros(q.shape, np.float64)
    s = np.einsum("...id,...jd->...ij", q, k) * scale
    s -= s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("...ij,...jd->...id", p, v)


def sdpa_math_fp32(q16, k16, v16, scale):
    """torch SDPA, MATH backend, CPU, on the fp32 upcast of the given tensors."""
    import torch
    from torch.nn.attention import SDPBackend, sdpa_kernel

    q = q16.detach().to("cpu", torch.float32)
    k = k16.detach().to("cpu", torch.float32)
    v = v16.detach().to("cpu", torch.float32)
    if k.shape[-2] == 0:
        return torch.zeros_like(q)
    with sdpa_kernel(SDPBackend.MATH):
        return torch.nn.functional.scaled_dot_product_attention(q, k, v, scale=scale)


def chunked_sdpa_math(q16, k16, v16, scale, rows=2048):
    """sdpa_math_fp32 computed per (b, h) and per block of `rows` query rows."""
    import torch

    B, H, Sq, D = q16.shape
    out = torch.empty((B, H, Sq, D), dtype=torch.float32)
    for b in range(B):
        for h in range(H):
            for r0 in range(0, Sq, rows):
                out[b, h, r0:r0 + rows] = sdpa_math_fp32(
                    q16[b, h, r0:r0 + rows], k16[b, h], v16[b, h], scale)
    return out


def online_softmax_tiled(q, k, v, scale, tile_n=16):
    """Streaming (online-softmax) attention over key tiles of `tile_n`, float64.

    Mirrors the reference's per-row state machine (attn_kernel.hip:357,
    :452-462, :486-492, :497-511) with every row of every head processed in
    parallel.
    """
    q, k, v = _as64(q), _as64(k), _as64(v)
    Skv = k.shape[-2]
    m = np.full(q.shape[:-1], -np.inf)
    l = np.zeros(q.shape[:-1])
    acc = np.zeros(q.shape[:-1] + (v.shape[-1],))
    for n0 in range(0, Skv, tile_n):
        kt, vt = k[..., n0:n0 + tile_n, :], v[..., n0:n0 + tile_n, :]
        s = np.einsum("...id,...jd->...ij", q, kt) * scale
        m_new = np.maximum(m, s.max(axis=-1))
        e = np.exp(s - m_new[..., None])
        rs = np.where(l > 0, np.exp(m - m_new), 0.0)
        acc = acc * rs[..., None] + np.einsum("...ij,...jd->...id", e, vt)
        l = l * rs + e.sum(axis=-1)
        m = m_new
    out = np.zeros_like(acc)
    live = l > 0
    out[live] = acc[live] / l[live][..., None]
    return out


def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


# Rescale limit of each kernel, as log2 of the largest p a block may carry
# on the running max before the exact block max is taken: D <= 64 keeps the
# exact running max (limit 2^0), D = 128 a lazy one (2^15), D = 512 2^8.
def kernel_tau(D):
    return 0.0 if D <= 64 else (15.0 if D == 128 else 8.0)


# Keys over which each kernel takes one rescale decision: the D <= 64 ring
# kernel raises its running max once per 64-key tile for up to 8192 keys and
# once per 32-key block above that; D = 128 tests each 32-key block and
# D = 512 each 32-key tile.
def kernel_tile(D, Skv):
    return 64 if D <= 64 and Skv <= 8192 else 32


# Query rows that share one rescale decision (the kernels' wave-uniform
# branch): the D = 128 kernel's wave of 32 rows; the D = 512 kernels decide
# per 16-row column block (per wave in attn_fwd_d512, per block in
# attn_fwd_d512w), and D <= 64 per 16-row column block, where with the exact
# running max the grouping changes nothing (a row whose max did not rise
# keeps m, and its rescale factor is exactly 1).
def kernel_wave_rows(D):
    return 32 if D == 128 else 16


def kernel_numerics_model(q16, k16, v16, scale, tau=None, tile_n=None, wave_rows=None):
    """The gfx950 kernel's arithmetic, restated in numpy (float32 state).

    Per block of `tile_n` keys: s = q.k in fp32; p = exp2(s*c - m) with the
    running max m (log2 units, c = |scale|*log2e), rounded to fp16. When some
    rounded p of the block exceeds 2^tau in any of the `wave_rows` rows that
    share a decision (the kernels' wave-uniform branch), each of those rows
    takes its exact block max: m' = max(m, max s*c), O and l scale by
    exp2(m - m') and P is recomputed. Then l += sum(p_fp16),
    acc += p_fp16 @ v; finally o = fp16(acc * (1/l)). tau, tile_n and
    wave_rows default to the kernel's choices for the head dim and key count
    (kernel_tau, kernel_tile, kernel_wave_rows). Negative scale is applied as
    (-q, |scale|), exact in fp16.
    """
    q = _as64(q16).astype(np.float32)
    k = _as64(k16).astype(np.float32)
    v = _as64(v16).astype(np.float32)
    if scale < 0:
        q = -q
    D = q.shape[-1]
    tau = kernel_tau(D) if tau is None else tau
    tile_n = kernel_tile(D, k.shape[-2]) if tile_n is None else tile_n
    wave_rows = kernel_wave_rows(D) if wave_rows is None else wave_rows
    c = np.float32(abs(scale) * LOG2E)
    lead, Sq, Skv = q.shape[:-2], q.shape[-2], k.shape[-2]
    m = np.full(q.shape[:-1], -1e30, np.float32)
    l = np.zeros(q.shape[:-1], np.float32)
    acc = np.zeros(q.shape[:-1] + (v.shape[-1],), np.float32)
    nw = -(-Sq // wave_rows)
    lim = np.float32(2.0 ** tau)
    for n0 in range(0, Skv, tile_n):
        s = np.einsum("...id,...jd->...ij", q, k[..., n0:n0 + tile_n, :]).astype(np.float32)
        with np.errstate(over="ignore"):  # p = inf on the first block (m = -1e30)
            p = _f16(np.exp2(s * c - m[..., None]))
        big = ~(p <= lim).all(axis=-1)                       # [..., Sq]
        pad = np.zeros(lead + (nw * wave_rows - Sq,), bool)
        wave = np.concatenate([big, pad], axis=-1).reshape(lead + (nw, wave_rows)).any(axis=-1)
        sel = np.repeat(wave, wave_rows, axis=-1)[..., :Sq]
        if sel.any():
            m_new = np.where(sel, np.maximum(m, s.max(axis=-1) * c), m).astype(np.float32)
            alpha = np.exp2(m - m_new).astype(np.float32)
            acc *= alpha[..., None]
            l *= alpha
            m = m_new
            p = _f16(np.exp2(s * c - m[..., None]))
        l += p.sum(axis=-1, dtype=np.float32)
        acc += np.einsum("...ij,...jd->...id", p, v[..., n0:n0 + tile_n, :]).astype(np.float32)
    out = np.zeros_like(acc)
    live = l > 0
    inv = (np.float32(1) / l[live]).astype(np.float32)
    out[live] = acc[live] * inv[..., None]
    return _f16(out)


def error_stats(out, ref):
    """(max-abs, mean-abs) error of `out` against `ref`, both cast to float64."""
    d = np.abs(_as64(out) - _as64(ref))
    if d.size == 0:
        return 0.0, 0.0
    return float(d.max()), float(d.mean())


def within_tolerance(out, ref, max_tol=MAX_ABS_TOL, mean_tol=MEAN_ABS_TOL):
    mx, mn = error_stats(out, ref)
    return mx <= max_tol and mn <= mean_tol, mx, mn


# Significant bits of the output formats (implicit bit included).
OUT_BITS = {"fp16": 11, "bf16": 8}


def round_to_format(x, fmt):
    """x (float64 array, finite, exactly representable in float32, as every
    fp32 reference is) rounded to the nearest `fmt` value, ties to even,
    returned as float64: fp16 through numpy's float16 (IEEE binary16,
    subnormals included), bf16 by keeping the upper 16 bits of the float32
    value with a round-to-nearest-even carry."""
    x = np.asarray(x, dtype=np.float64)
    if fmt == "fp16":
        with np.errstate(over="ignore"):  # beyond 65504: inf, as the hardware's conversion
            return x.astype(np.float16).astype(np.float64)
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32).astype(np.float64)


def within_rounded_tolerance(out, ref, fmt="fp16", mult=1.0):
    """The north-star bars (times `mult`) for an output stored in `fmt`, where
    that format's own spacing allows them.

    Element by element, the error may instead reach half a unit in the last
    place of `ref` in `fmt` plus the mean bar: an fp16 output with |o| >= 4
    errs by up to 1.95e-3 when correctly rounded, so an absolute 2e-3 would
    leave 5e-5 for everything before the rounding; below 4 (fp16) the bar is
    the plain one. The mean error may instead reach that of `ref` correctly
    rounded to `fmt` plus half the mean bar: a few bf16 outputs near 1 carry a
    mean rounding error of about 1e-3 on their own (half an ulp there is
    3.9e-3), most of bf16's 1.6e-3 mean bar. Returns (ok, max-abs, mean-abs)."""
    o, r = _as64(out), _as64(ref)
    d = np.abs(o - r)
    if d.size == 0:
        return True, 0.0, 0.0
    _, e = np.frexp(np.abs(r))  # |r| = f * 2^e, f in [0.5, 1)
    half_ulp = np.ldexp(1.0, np.maximum(e - OUT_BITS[fmt] - 1, -149))
    allowed = np.maximum(half_ulp + mult * MEAN_ABS_TOL, mult * MAX_ABS_TOL)
    rounded = round_to_format(r, fmt)
    floor = np.where(np.isfinite(rounded), np.abs(rounded - r), half_ulp)  # past fp16's range
    floor_mean = float(floor.mean())
    mean_allowed = max(mult * MEAN_ABS_TOL, floor_mean + 0.5 * mult * MEAN_ABS_TOL)
    return bool((d <= allowed).all()) and float(d.mean()) <= mean_allowed, \
        float(d.max()), float(d.mean())


# ---------------------------------------------------------------------------
# Workloads and seeded inputs.

CONFIGS = {
    # name: (B, H, Sq, Skv, D, q/k multiplier, v multiplier, seed)
    "c1": (1, 1, 1024, 1024, 64, 1.0, 1.0, 101),
    "c2": (1, 16, 4096, 4096, 128, 1.0, 1.0, 102),
    "c3": (2, 24, 8192, 512, 64, 2.0, 1.0, 103),
    "c4": (1, 4, 8192, 8192, 512, 0.5, 0.5, 104),
    "c5": (1, 8, 131072, 131072, 64, 1.0, 1.0, 105),
    "ns": (1, 16, 16384, 16384, 128, 1.0, 1.0, 106),
}


def make_inputs(B, H, Sq, Skv, D, qk_mult=1.0, v_mult=1.0, seed=0):
    """fp16 q [B,H,Sq,D], k/v [B,H,Skv,D] on CPU: N(0,1) fp32 from a seeded
    CPU generator, times the multiplier, then rounded to fp16."""
    import torch

    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, H, Sq, D, generator=g) * qk_mult).half()
    k = (torch.randn(B, H, Skv, D, generator=g) * qk_mult).half()
    v = (torch.randn(B, H, Skv, D, generator=g) * v_mult).half()
    return q, k, v


def config_inputs(name):
    B, H, Sq, Skv, D, qm, vm, seed = CONFIGS[name]
    return make_inputs(B, H, Sq, Skv, D, qm, vm, seed)


def time_cpu_sdpa(q16, k16, v16, scale, reps=3):
    """Min-of-`reps` wall time (s) of chunked_sdpa_math after one warm-up."""
    chunked_sdpa_math(q16, k16, v16, scale)
    best = math.inf
    for _ in range(reps):
        t0 = time.perf_counter()
        chunked_sdpa_math(q16, k16, v16, scale)
        best = min(best, time.perf_counter() - t0)
    return best
