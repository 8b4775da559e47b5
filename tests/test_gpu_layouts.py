"""Native bf16 and strided layouts on the GPU.

bf16: parity against torch SDPA MATH in fp32 on the same bf16 inputs. bf16
keeps 8 significand bits to fp16's 11, so the fp16 bars (2e-3 / 2e-4) are
scaled by 8; as for fp16, where |ref| is so large that the bf16 spacing
alone exceeds the bar, the output must be the bf16 rounding of a value
within the mean bar of the reference.

Strides: the kernel reads [B, H, S, D] views with any batch / head /
sequence strides in place. Every strided call is compared bit for bit with
the same call on contiguous copies (same arithmetic on the same values), both
through the C ABI (explicit strides) and through the torch op (which passes
strides instead of copying).
"""

import ctypes

import pytest
import torch

import gfx906_amd
from oracle.attention import make_inputs, sdpa_math_fp32

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF16_MAX_ABS, BF16_MEAN_ABS = 8 * 2e-3, 8 * 2e-4
ATTN_DTYPE_F16, ATTN_DTYPE_BF16 = 0, 1


def bf16_half_ulp(x):
    """Half the bf16 spacing at |x|."""
    _, e = torch.frexp(x.abs())  # |x| = m * 2^e, m in [0.5, 1)
    return torch.ldexp(torch.ones_like(x), (e - 9).clamp(min=-133))


def assert_close_bf16(out, ref, what):
    d = (out.float().cpu() - ref).abs()
    mx, mn = d.max().item(), d.mean().item()
    print(f"{what}: max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)
    allowed = torch.clamp(bf16_half_ulp(ref) + BF16_MEAN_ABS, min=BF16_MAX_ABS)
    assert bool((d <= allowed).all()) and mn <= BF16_MEAN_ABS, (what, mx, mn)


def bf16_inputs(B, H, Sq, Skv, D, seed, qk_mult=1.0):
    return tuple(t.to(torch.bfloat16) for t in make_inputs(B, H, Sq, Skv, D, qk_mult, 1.0, seed))


def capi_ex(q, k, v, o, scale, dtype, strides=None):
    """attn_fwd_ex through ctypes; strides: dict name -> (b, h, s) or None."""
    lib = gfx906_amd.capi()
    B, H, Sq, D = q.shape
    arrs = []
    for name in "qkvo":
        s = (strides or {}).get(name)
        arrs.append(None if s is None else (ctypes.c_longlong * 3)(*s))
    rc = lib.attn_fwd_ex(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H, Sq,
                         k.shape[2], D, float(scale), torch.cuda.current_stream().cuda_stream,
                         dtype, *arrs)
    torch.cuda.synchronize()
    return rc, lib.attn_last_error()


# -- bf16 -------------------------------------------------------------------------------

@pytest.mark.parametrize("D,Sq,Skv", [(128, 300, 517), (64, 257, 130), (40, 100, 77),
                                      (512, 140, 96), (128, 1, 1), (64, 64, 1000)])
def test_bf16_matches_sdpa(D, Sq, Skv):
    q, k, v = bf16_inputs(2, 3, Sq, Skv, D, seed=D + Sq + Skv)
    out = gfx906_amd.attn(q.to(DEV), k.to(DEV), v.to(DEV), D ** -0.5)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16 and out.shape == q.shape
    assert_close_bf16(out, sdpa_math_fp32(q, k, v, D ** -0.5), f"bf16 D{D} Sq{Sq} Skv{Skv}")


@pytest.mark.parametrize("D", [128, 64, 512])
def test_bf16_sharp_and_negative_scale(D):
    q, k, v = bf16_inputs(1, 2, 200, 333, D, seed=D + 5, qk_mult=2.0)
    for scale in (D ** -0.5, -(D ** -0.5)):
        out = gfx906_amd.attn(q.to(DEV), k.to(DEV), v.to(DEV), scale)
        assert_close_bf16(out, sdpa_math_fp32(q, k, v, scale), f"bf16 D{D} scale {scale:.3g}")


def test_bf16_capi_matches_binding():
    q, k, v = (t.to(DEV) for t in bf16_inputs(2, 4, 150, 260, 128, seed=3))
    a = gfx906_amd.attn(q, k, v, 0.1)
    o = torch.empty_like(q)
    rc, err = capi_ex(q, k, v, o, 0.1, ATTN_DTYPE_BF16)
    assert rc == 0, err
    assert torch.equal(a, o)


def test_bf16_single_key_returns_v0():
    q, k, v = bf16_inputs(1, 2, 40, 1, 64, seed=8)
    out = gfx906_amd.attn(q.to(DEV), k.to(DEV), v.to(DEV), 0.2).cpu()
    assert torch.equal(out, v.expand_as(out))


def test_dtype_mismatch_rejected():
    q = torch.zeros(1, 1, 8, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="dtype"):
        gfx906_amd.attn(q, q.half(), q.half(), 0.1)


# -- strides: C ABI ---------------------------------------------------------------------

def bshd_view(t):
    """The same values as t ([B,H,S,D]) stored as [B,S,H,D], viewed as [B,H,S,D]."""
    return t.transpose(1, 2).contiguous().transpose(1, 2)


def strides_of(t):
    return tuple(t.stride(i) for i in range(3))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [128, 64, 24, 512])
def test_capi_bshd_layout_bit_exact(dtype, D):
    q, k, v = (t.to(dtype).to(DEV) for t in make_inputs(2, 3, 130, 201, D, seed=D + 40))
    ref = torch.empty_like(q)
    code = ATTN_DTYPE_BF16 if dtype == torch.bfloat16 else ATTN_DTYPE_F16
    rc, err = capi_ex(q, k, v, ref, D ** -0.5, code)
    assert rc == 0, err
    qs, ks, vs = bshd_view(q), bshd_view(k), bshd_view(v)
    obuf = torch.full((2, 130, 3, D), float("nan"), dtype=dtype, device=DEV)
    o = obuf.transpose(1, 2)
    rc, err = capi_ex(qs, ks, vs, o, D ** -0.5, code,
                      {"q": strides_of(qs), "k": strides_of(ks), "v": strides_of(vs),
                       "o": strides_of(o)})
    assert rc == 0, err
    assert torch.equal(o, ref)


def test_capi_broadcast_kv_over_heads():
    # k/v of one head shared by all heads: head stride 0.
    q, k, v = (t.to(DEV) for t in make_inputs(2, 4, 96, 150, 128, seed=41))
    k1, v1 = k[:, :1], v[:, :1]
    ref = torch.empty_like(q)
    rc, err = capi_ex(q, k1.expand_as(k).contiguous(), v1.expand_as(v).contiguous(), ref, 0.1,
                      ATTN_DTYPE_F16)
    assert rc == 0, err
    o = torch.empty_like(q)
    kst = (k1.stride(0), 0, k1.stride(2))
    rc, err = capi_ex(q, k1, v1, o, 0.1, ATTN_DTYPE_F16, {"k": kst, "v": kst})
    assert rc == 0, err
    assert torch.equal(o, ref)


def test_capi_sequence_stride():
    # Every other query row and key of larger tensors (sequence stride 2*D).
    q, k, v = (t.to(DEV) for t in make_inputs(1, 2, 200, 300, 64, seed=42))
    qs, ks, vs = q[:, :, ::2], k[:, :, ::2], v[:, :, ::2]
    ref = torch.empty(qs.shape, dtype=q.dtype, device=DEV)
    rc, err = capi_ex(qs.contiguous(), ks.contiguous(), vs.contiguous(), ref, 0.125,
                      ATTN_DTYPE_F16)
    assert rc == 0, err
    o = torch.empty_like(ref)
    rc, err = capi_ex(qs, ks, vs, o, 0.125, ATTN_DTYPE_F16,
                      {"q": strides_of(qs), "k": strides_of(ks), "v": strides_of(vs)})
    assert rc == 0, err
    assert torch.equal(o, ref)


# -- strides: torch op ------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_op_reads_bshd_views_and_writes_out(dtype):
    q, k, v = (t.to(dtype).to(DEV) for t in make_inputs(2, 4, 300, 257, 128, seed=43))
    ref = gfx906_amd.attn(q, k, v, 0.09)
    buf = torch.empty(2, 300, 4, 128, dtype=dtype, device=DEV)
    out = gfx906_amd.attn(bshd_view(q), bshd_view(k), bshd_view(v), 0.09, out=buf.transpose(1, 2))
    torch.cuda.synchronize()
    assert out.data_ptr() == buf.data_ptr()
    assert torch.equal(buf.transpose(1, 2), ref)


def test_op_broadcast_and_unaligned_views():
    q, k, v = (t.to(DEV) for t in make_inputs(1, 3, 77, 90, 64, seed=44))
    ref = gfx906_amd.attn(q, k[:, :1].expand_as(k).contiguous(), v[:, :1].expand_as(v).contiguous(),
                          0.125)
    assert torch.equal(gfx906_amd.attn(q, k[:, :1].expand_as(k), v[:, :1].expand_as(v), 0.125),
                       ref)
    # A view starting 4 elements into its storage is not 16-byte aligned: copied, same result.
    big = torch.zeros(q.numel() + 4, dtype=q.dtype, device=DEV)
    big[4:] = q.flatten()
    qu = big[4:].view_as(q)
    assert qu.data_ptr() % 16 != 0
    ref2 = gfx906_amd.attn(q, k, v, 0.125)
    assert torch.equal(gfx906_amd.attn(qu, k, v, 0.125), ref2)


def test_op_out_may_be_q():
    q, k, v = (t.to(DEV) for t in make_inputs(1, 2, 333, 100, 128, seed=45))
    ref = gfx906_amd.attn(q, k, v, 0.1)
    qq = q.clone()
    out = gfx906_amd.attn(qq, k, v, 0.1, out=qq)
    torch.cuda.synchronize()
    assert out.data_ptr() == qq.data_ptr() and torch.equal(qq, ref)


def test_op_out_rejections():
    q = torch.zeros(1, 2, 16, 64, dtype=torch.float16, device=DEV)
    with pytest.raises(RuntimeError, match="overlap"):
        gfx906_amd.attn(q, q, q, 0.1, out=torch.empty(1, 2, 1, 64, dtype=q.dtype,
                                                     device=DEV).expand(1, 2, 16, 64))
    with pytest.raises(RuntimeError, match="dtype"):
        gfx906_amd.attn(q, q, q, 0.1, out=torch.empty_like(q, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match=r"\[B, H, Sq, D\]"):
        gfx906_amd.attn(q, q, q, 0.1, out=torch.empty(1, 2, 15, 64, dtype=q.dtype, device=DEV))
    with pytest.raises(RuntimeError, match="contiguous head dim"):
        gfx906_amd.attn(q, q, q, 0.1,
                        out=torch.empty(1, 2, 64, 16, dtype=q.dtype, device=DEV).transpose(2, 3))
