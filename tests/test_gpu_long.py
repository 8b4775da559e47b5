"""Long sequences on the GPU: the reference's long-context checks.

* D = 512 at S = 129,600 tokens (bench_d512.py:63-79, README.md:5 "129K
  verified"): a seeded 512-row query slice against the CPU oracle on the
  full K/V, through the torch op.
* D = 64, B1 H8 S = 32,768 (test.py:48-61, the "memory-bound proof"): a
  256-row slice against the oracle.

Both also check that the op's peak device memory stays O(S*D): the output
plus at most a small workspace, never an S x S score matrix (which would be
67 GB at S = 129,600 and 34 GB at S = 32,768 in fp32).
"""

import pytest
import torch

import gfx906_amd
from oracle.attention import MAX_ABS_TOL, MEAN_ABS_TOL, error_stats, make_inputs, sdpa_math_fp32

pytestmark = pytest.mark.gpu


def _run_and_peak(q, k, v, scale):
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    out = gfx906_amd.attn(q, k, v, scale)
    torch.cuda.synchronize()
    return out, torch.cuda.max_memory_allocated() - base


def _slice_check(q, k, v, out, scale, n, seed, what):
    g = torch.Generator().manual_seed(seed)
    rows = torch.randperm(q.shape[2], generator=g)[:n].sort().values
    ref = sdpa_math_fp32(q[:, :, rows], k, v, scale)
    mx, mn = error_stats(out[:, :, rows].float().cpu(), ref)
    print(f"{what}: {n}-row slice max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)
    assert mx <= MAX_ABS_TOL and mn <= MEAN_ABS_TOL, (what, mx, mn)
    assert torch.isfinite(out.float()).all()


def test_d512_129600_tokens():
    S, D = 129_600, 512  # not a multiple of the 128-row query tile: ragged last tile
    print(f"case: B1 H1 S{S} D{D}", flush=True)
    q, k, v = make_inputs(1, 1, S, S, D, seed=129)
    scale = D ** -0.5
    out, peak = _run_and_peak(q.cuda(), k.cuda(), v.cuda(), scale)
    tensor_bytes = S * D * 2
    print(f"peak device memory above inputs: {peak / 2**20:.1f} MiB "
          f"(one S x D tensor: {tensor_bytes / 2**20:.1f} MiB)", flush=True)
    assert peak <= 2 * tensor_bytes
    _slice_check(q, k, v, out.cpu(), scale, 512, seed=1296, what="S=129600 D=512")


def test_d64_32768_tokens_memory():
    B, H, S, D = 1, 8, 32_768, 64
    print(f"case: B{B} H{H} S{S} D{D}", flush=True)
    q, k, v = make_inputs(B, H, S, S, D, seed=327)
    out, peak = _run_and_peak(q.cuda(), k.cuda(), v.cuda(), 0.125)
    tensor_bytes = B * H * S * D * 2
    print(f"peak device memory above inputs: {peak / 2**20:.1f} MiB "
          f"(one output: {tensor_bytes / 2**20:.1f} MiB)", flush=True)
    assert peak <= 2 * tensor_bytes
    _slice_check(q, k, v, out.cpu(), 0.125, 256, seed=3276, what="S=32768 D=64")
