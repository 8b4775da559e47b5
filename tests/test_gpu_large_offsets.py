"""Views that lie past the first 4 GiB of their allocation: 64-bit addressing.

An MI355X holds 288 GB, so a caller's q, k, v or o may start far into a
large allocation (a big batch, a packed activation or KV buffer). The
kernels form each head's and each tile's base address in 64 bits and keep
32-bit offsets only inside one tile's buffer range. Each case here places
batch 1 of q, k, v and o more than 2^32 bytes after batch 0 (batch stride
2^31 + 2^16 elements, in two 4 GiB buffers) and checks that

* the output equals, bit for bit, the same call on the same layout with a
  small batch stride,
* seeded rows meet the parity bar against SDPA MATH in fp32 on the CPU,
* nothing outside the output view is written (NaN sentinels after batch 0,
  before and after batch 1).

Split key ranges (small grids), whole grids, Q through LDS (more than 1024
keys), D = 512 with row-major and token-contiguous K/V are covered. Each
case prints its parameters first.
"""

import pytest
import torch

import gfx906_amd
from oracle.attention import MAX_ABS_TOL, MEAN_ABS_TOL, error_stats, make_inputs, sdpa_math_fp32

pytestmark = pytest.mark.gpu

BIG_STRIDE = (1 << 31) + (1 << 16)  # elements: batch 1 starts 4 GiB + 128 KiB in
SLAB = 1 << 24  # elements of one batch that a case's tensors may fill
CASES = [  # B, H, Sq, Skv, D, k/v layout
    (2, 2, 300, 1100, 64, "rows"),  # split key range
    (2, 4, 16384, 260, 64, "rows"),  # whole grid, two workgroups per CU
    (2, 2, 300, 1100, 128, "rows"),  # split key range
    (2, 2, 16384, 1100, 128, "rows"),  # whole grid, Q through LDS
    (2, 1, 300, 1100, 512, "rows"),  # split key range
    (2, 2, 8192, 96, 512, "rows"),  # whole grid (32 query rows per wave)
    (2, 1, 1024, 1024, 512, "tokens"),  # token-contiguous k/v read in place
]


def packed_views(buf, shapes, batch_stride, tokens_kv):
    """Views of `buf` with the given [B, H, S, D] shapes, one after another
    inside each batch's slab; batch b of every view starts at b * batch_stride.
    With tokens_kv the second and third views (k, v) keep the sequence
    contiguous and the head dim S apart, as a [b, c, h*w] activation does."""
    views, base = [], 0
    for i, (B, H, S, D) in enumerate(shapes):
        if tokens_kv and i > 0:
            assert H == 1
            strides = (batch_stride, S * D, 1, S)
        else:
            strides = (batch_stride, S * D, D, 1)
        views.append(buf.as_strided((B, H, S, D), strides, base))
        base += -(-H * S * D // 64) * 64
    assert base <= SLAB
    return views


@pytest.fixture(scope="module")
def buffers():
    need = 2 * 2 * (BIG_STRIDE + SLAB) + 4 * 2 * SLAB  # bytes: two big, two small buffers
    if torch.cuda.mem_get_info()[0] < need + (4 << 30):
        pytest.skip("not enough free device memory for two 4 GiB buffers")
    bufs = [torch.empty(BIG_STRIDE + SLAB, dtype=torch.float16, device="cuda") for _ in range(2)]
    bufs += [torch.empty(2 * SLAB, dtype=torch.float16, device="cuda") for _ in range(2)]
    yield bufs
    bufs.clear()
    torch.cuda.empty_cache()


@pytest.mark.parametrize("B,H,Sq,Skv,D,kv_layout", CASES)
def test_views_past_4gib(buffers, B, H, Sq, Skv, D, kv_layout):
    print(f"case {kv_layout}: B{B} H{H} Sq{Sq} Skv{Skv} D{D}", flush=True)
    big_in, big_out, small_in, small_out = buffers
    tokens = kv_layout == "tokens"
    q, k, v = make_inputs(B, H, Sq, Skv, D, 1.0, 1.0, 11)
    scale = D ** -0.5
    shapes = [tuple(q.shape), tuple(k.shape), tuple(v.shape)]
    outs = []
    for buf_in, buf_out, stride in ((big_in, big_out, BIG_STRIDE), (small_in, small_out, SLAB)):
        qv, kv, vv = packed_views(buf_in, shapes, stride, tokens)
        for dst, src in ((qv, q), (kv, k), (vv, v)):
            dst.copy_(src.cuda())
        buf_out.fill_(float("nan"))
        (ov,) = packed_views(buf_out, shapes[:1], stride, False)
        res = gfx906_amd.attn(qv, kv, vv, scale, out=ov)
        assert res.data_ptr() == ov.data_ptr()
        outs.append(ov)
    torch.cuda.synchronize()
    far, near = outs
    # batch 1 of every view lies past the first 2^32 bytes of its buffer
    assert BIG_STRIDE * 2 > (1 << 32)
    assert torch.isfinite(far).all()
    assert torch.equal(far, near)
    n = H * Sq * D
    for lo in (n, BIG_STRIDE - 4096, BIG_STRIDE + n):
        assert torch.isnan(big_out[lo:lo + 4096]).all(), lo
    rows = torch.cat([torch.arange(64), torch.arange(Sq - 64, Sq)]) if Sq > 128 else torch.arange(Sq)
    ref = sdpa_math_fp32(q[:, :, rows], k, v, scale)
    mx, mn = error_stats(far[:, :, rows.cuda()].float().cpu(), ref)
    print(f"  far == near; {len(rows)} rows per head: max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)
    assert mx <= MAX_ABS_TOL and mn <= MEAN_ABS_TOL
