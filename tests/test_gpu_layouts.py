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
from oracle.attention import within_tolerance, make_inputs, sdpa_math_fp32

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
    """attn_fwd_ex through ctypes; strides: dict name -> (b, h, s[, d]) or None
    (d = 1 when omitted)."""
    lib = gfx906_amd.capi()
    B, H, Sq, D = q.shape
    arrs = []
    for name in "qkvo":
        s = (strides or {}).get(name)
        arrs.append(None if s is None else
                    (ctypes.c_longlong * 4)(*s, *((1,) if len(s) == 3 else ())))
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


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D,Skv", [(64, 201), (128, 201), (512, 201), (512, 4100)])
def test_capi_output_rows_not_16_byte_aligned(dtype, D, Skv):
    # Output rows D + 4 elements apart (8-byte aligned, not 16): the kernels
    # store such rows directly instead of staging whole rows through LDS; the
    # result must equal the contiguous output bit for bit (Skv = 4100 at
    # D = 512 also takes the split key range path).
    q, k, v = (t.to(dtype).to(DEV) for t in make_inputs(1, 3, 150, Skv, D, seed=D + 45))
    code = ATTN_DTYPE_BF16 if dtype == torch.bfloat16 else ATTN_DTYPE_F16
    lib = gfx906_amd.capi()
    need = lib.attn_split_workspace_bytes(1, 3, 150, Skv, D)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    padded = torch.full((1, 3, 150, D + 4), float("nan"), dtype=dtype, device=DEV)
    outs = []
    for o in (torch.empty_like(q), padded[..., :D]):
        st = lambda t: (ctypes.c_longlong * 4)(*[t.stride(i) for i in range(4)])
        rc = lib.attn_fwd_split(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), 1, 3, 150,
                                Skv, D, D ** -0.5, stream, code, None, None, None, st(o),
                                ctypes.c_void_p(ws.data_ptr()), need)
        assert rc == 0, lib.attn_last_error()
        outs.append(o)
    torch.cuda.synchronize()
    assert (need > 0) == (Skv == 4100)
    assert torch.equal(outs[1], outs[0])
    assert torch.isnan(padded[..., D:]).all()  # the padding is untouched


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


def test_op_out_with_strided_head_dim_is_filled():
    # Outside the token-contiguous D = 512 case the kernel writes a temporary
    # that is then copied into `out`.
    q, k, v = (t.to(DEV) for t in make_inputs(1, 2, 16, 40, 64, seed=46))
    ref = gfx906_amd.attn(q, k, v, 0.1)
    buf = torch.empty(1, 2, 64, 16, dtype=q.dtype, device=DEV)
    out = gfx906_amd.attn(q, k, v, 0.1, out=buf.transpose(2, 3))
    torch.cuda.synchronize()
    assert out.data_ptr() == buf.data_ptr() and torch.equal(buf.transpose(2, 3), ref)


# -- token-contiguous D = 512 (the VAE's [b, c, h*w] activations) ------------------------

def assert_near(got, ref, dtype):
    """Token-contiguous vs contiguous kernel: same math, another summation order
    inside each 32-key block; the difference stays within the parity bar."""
    d = (got.float() - ref.float()).abs().max().item()
    print(f"token-contiguous vs contiguous: max-abs {d:.2e}", flush=True)
    assert d <= (2e-3 if dtype == torch.float16 else 1.6e-2), d


def vae_views(x):
    """[b, c, h, w] -> the [b, 1, h*w, c] view the VAE hook hands the kernel
    (deploy/gfx906_attention.py:102-104): sequence stride 1, head-dim stride h*w."""
    b, c, h, w = x.shape
    return x.reshape(b, c, h * w).transpose(1, 2).unsqueeze(1)


def tl_strides(t):
    """{batch, head, seq, head dim} strides, 0 for the size-1 batch/head dims."""
    return tuple(0 if t.size(d) == 1 and d < 3 else t.stride(d) for d in range(4))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("b,h,w", [(1, 8, 8), (2, 16, 24), (1, 32, 33), (1, 64, 64)])
def test_token_contiguous_d512_in_place_via_capi(dtype, b, h, w):
    # The kernel reads [b, 1, h*w, c] views of [b, c, h, w] tensors and writes
    # such a view of the output, with no copy and no allocation.
    g = torch.Generator().manual_seed(b * 1000 + h * 10 + w)
    xs = [(torch.randn(b, 512, h, w, generator=g) * m).to(dtype).to(DEV)
          for m in (0.5, 0.5, 1.0)]
    qv, kv, vv = (vae_views(x) for x in xs)
    assert kv.stride(2) == 1 and kv.stride(3) == h * w
    ref = gfx906_amd.attn(qv.contiguous(), kv.contiguous(), vv.contiguous(), 512 ** -0.5)
    out = torch.empty(b, 512, h, w, dtype=dtype, device=DEV)
    ov = vae_views(out)
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    rc, err = capi_ex(qv, kv, vv, ov, 512 ** -0.5,
                      ATTN_DTYPE_F16 if dtype == torch.float16 else ATTN_DTYPE_BF16,
                      {n: tl_strides(t) for n, t in zip("qkvo", (qv, kv, vv, ov))})
    assert rc == 0, err
    assert torch.cuda.max_memory_allocated() == base
    # the same arithmetic as the contiguous kernel, with the keys of each
    # 32-key MFMA summed in another order: equal to within fp16/bf16 rounding
    assert_near(ov, ref, dtype)
    if dtype == torch.float16 and h * w <= 1024:
        exact = sdpa_math_fp32(qv.float().cpu(), kv.float().cpu(), vv.float().cpu(), 512 ** -0.5)
        ok, mx, mn = within_tolerance(ov.float().cpu(), exact)
        assert ok, (mx, mn)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("h,w", [(12, 20), (72, 72), (96, 96)])
def test_op_vae_views_and_nchw_out(dtype, h, w):
    # The torch op on the VAE's views, written through a [b, c, h, w] view:
    # read in place up to 6400 tokens (no allocation beyond the split
    # workspace), copied above.
    g = torch.Generator().manual_seed(3)
    xs = [(torch.randn(1, 512, h, w, generator=g) * 0.5).to(dtype).to(DEV) for _ in range(3)]
    qv, kv, vv = (vae_views(x) for x in xs)
    ref = gfx906_amd.attn(qv.contiguous(), kv.contiguous(), vv.contiguous(), 512 ** -0.5)
    out = torch.empty_like(xs[0])
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    got = gfx906_amd.attn(qv, kv, vv, 512 ** -0.5, out=vae_views(out))
    torch.cuda.synchronize()
    ws = gfx906_amd.capi().attn_split_workspace_bytes(1, 1, h * w, h * w, 512)
    copies = 4 * h * w * 512 * 2
    extra = torch.cuda.max_memory_allocated() - base
    if h * w <= 6400:  # only the split workspace (allocator blocks of 512 bytes)
        assert extra <= (ws + 511) // 512 * 512, (extra, ws)
    else:
        assert extra >= copies, (extra, copies)
    assert got.data_ptr() == out.data_ptr()
    assert_near(vae_views(out), ref, dtype)


def test_token_contiguous_with_q_head_dim_stride_2():
    # The reference's own non-contiguous case (test_d512.py:22-30): q a
    # [:, :, ::2] view, k and v transposed [b, D, S] tensors.
    g = torch.Generator().manual_seed(7)
    S, D = 1024, 512
    q = torch.randn(1, S, 2 * D, generator=g).half().to(DEV)[:, :, ::2].unsqueeze(1)
    k = torch.randn(1, D, S, generator=g).half().to(DEV).transpose(1, 2).unsqueeze(1)
    v = torch.randn(1, D, S, generator=g).half().to(DEV).transpose(1, 2).unsqueeze(1)
    ref = gfx906_amd.attn(q.contiguous(), k.contiguous(), v.contiguous(), D ** -0.5)
    assert_near(gfx906_amd.attn(q, k, v, D ** -0.5), ref, torch.float16)  # read in place
    o = torch.empty_like(ref)
    rc, err = capi_ex(q, k, v, o, D ** -0.5, ATTN_DTYPE_F16,
                      {n: tl_strides(t) for n, t in zip("qkvo", (q, k, v, o))})
    assert rc == 0, err
    assert_near(o, ref, torch.float16)


def test_token_contiguous_heads_and_batches_via_capi():
    # [B, H, D, S] tensors seen as [B, H, S, D]: per-head K^T blocks.
    B, H, S, Sq, D = 2, 3, 200, 72, 512
    g = torch.Generator().manual_seed(9)
    kt = (torch.randn(B, H, D, S, generator=g) * 0.5).half().to(DEV)
    vt = torch.randn(B, H, D, S, generator=g).half().to(DEV)
    q = (torch.randn(B, H, Sq, D, generator=g) * 0.5).half().to(DEV)
    k, v = kt.transpose(2, 3), vt.transpose(2, 3)
    ref = torch.empty_like(q)
    rc, err = capi_ex(q, k.contiguous(), v.contiguous(), ref, 0.05, ATTN_DTYPE_F16)
    assert rc == 0, err
    o = torch.empty(B, H, D, Sq, dtype=q.dtype, device=DEV).transpose(2, 3)
    st = tuple(k.stride())
    rc, err = capi_ex(q, k, v, o, 0.05, ATTN_DTYPE_F16,
                      {"k": st, "v": st, "o": tuple(o.stride())})
    assert rc == 0, err
    assert_near(o, ref, torch.float16)


def test_token_contiguous_skv_not_multiple_of_8_is_rejected_by_capi():
    g = torch.Generator().manual_seed(11)
    x = [torch.randn(1, 512, 7, 9, generator=g).half().to(DEV) for _ in range(3)]  # hw = 63
    qv, kv, vv = (vae_views(t) for t in x)
    ref = gfx906_amd.attn(qv.contiguous(), kv.contiguous(), vv.contiguous(), 0.04)
    assert torch.equal(gfx906_amd.attn(qv, kv, vv, 0.04), ref)  # the op copies
    # through the C ABI: 63 tokens of rows padded to 64 (head-dim stride 64)
    kp = torch.randn(1, 512, 64, generator=g).half().to(DEV)[:, :, :63]
    kpv = kp.transpose(1, 2).unsqueeze(1)
    st = (kpv.stride(0), 0, 1, 64)  # the size-1 head dim's stride is unused: 0
    rc, err = capi_ex(qv.contiguous(), kpv, kpv, torch.empty_like(ref), 0.04, ATTN_DTYPE_F16,
                      {"k": st, "v": st})
    assert rc == 1 and b"Skv % 8" in err
