"""The reference's own conv3d kernel (hip_conv/conv3d_kernel.hip), built
unmodified for gfx950 into oracle/_ref/, as a second checker and a timing
reference.

On the reference's own cases (test_conv3d.py:58-69) its output agrees with
oracle.conv3d within the reference's bar (allclose atol=rtol=2e-2,
test_conv3d.py:29-34), and so does the gfx950 kernel's with it. On a VAE-sized
layer (512 -> 512 channels, 3x3x3) both are timed on the same GPU; the gfx950
kernel must be faster than the reference's. (torch's own conv3d is not timed:
its first call at this shape spends minutes in MIOpen's kernel search here.)
Skipped when oracle/_ref was not built (no /root/reference at build time).
"""

import ctypes
import os

import numpy as np
import pytest
import torch

from gfx906_amd import kitchen
from oracle import conv3d as oc

pytestmark = pytest.mark.gpu

REF_LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle",
                       "_ref", "libref_conv3d.so")
CL = torch.channels_last_3d


@pytest.fixture(scope="module")
def ref():
    if not os.path.isfile(REF_LIB):
        pytest.skip("oracle/_ref/libref_conv3d.so not built")
    lib = ctypes.CDLL(REF_LIB)
    lib.launch_conv3d.restype = None
    return lib


def run_ref(lib, x, w, bias, res, stride):
    n, c, d, h, ww = x.shape
    k, _, t, r, s = w.shape
    Z, P, Q = oc.output_size(d, h, ww, t, r, s, stride)
    out = torch.empty((n, k, Z, P, Q), dtype=torch.float16, device=x.device,
                      memory_format=CL)
    xs, os_ = kitchen.packed_strides(x.shape), kitchen.packed_strides(out.shape)
    rs = os_ if res is not None else (0, 0, 0, 0)
    ptr = [ctypes.c_void_p(0 if t_ is None else t_.data_ptr()) for t_ in (x, w, bias, res, out)]
    lib.launch_conv3d(*ptr, *[ctypes.c_int(v) for v in (n, d, h, ww, c, k, t, r, s, *stride,
                                                         Z, P, Q)],
                      ctypes.c_long(n * Z * P * Q), *[ctypes.c_long(v) for v in (*xs, *os_, *rs)],
                      ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    return out


def dev_case(i):
    xs, ws, stride, has_b, has_r = oc.REF_CASES[i]
    x, w, b, res = oc.make_case(xs, ws, stride, has_b, has_r, seed=300 + i)
    t = lambda a, fmt=CL: None if a is None else torch.from_numpy(a).cuda().contiguous(  # noqa: E731
        memory_format=fmt)
    return (x, w, b, res, stride), (t(x), t(w), None if b is None else torch.from_numpy(b).cuda(),
                                    t(res), stride)


@pytest.mark.parametrize("i", range(len(oc.REF_CASES)))
def test_reference_conv3d_agrees_with_oracle_and_ours(ref, i):
    (x, w, b, res, stride), (xd, wd, bd, rd, _) = dev_case(i)
    o_ref = run_ref(ref, xd, wd, bd, rd, stride)
    o_new = kitchen.try_kernel(xd, wd, bd, rd, list(stride))
    torch.cuda.synchronize()
    exact = torch.from_numpy(oc.conv3d_gemm(x, w, b, res, stride))
    r, nw = o_ref.double().cpu(), o_new.double().cpu()
    print(f"case{i}: reference vs oracle {(r - exact).abs().max().item():.2e}, "
          f"gfx950 vs reference {(nw - r).abs().max().item():.2e}", flush=True)
    assert torch.allclose(r, exact, atol=2e-2, rtol=2e-2)
    assert torch.allclose(nw, r, atol=2e-2, rtol=2e-2)


def _time(fn, reps=10):
    fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ts = []
    for _ in range(reps):
        a.record()
        fn()
        b.record()
        b.synchronize()
        ts.append(a.elapsed_time(b))
    return min(ts)


def test_vae_layer_timing(ref):
    g = np.random.default_rng(7)
    x = torch.from_numpy((g.standard_normal((1, 512, 8, 64, 64)) * 0.25).astype(np.float16))
    w = torch.from_numpy((g.standard_normal((512, 512, 3, 3, 3)) * 0.25).astype(np.float16))
    b = torch.from_numpy(g.standard_normal(512).astype(np.float16)).cuda()
    xd, wd = x.cuda().contiguous(memory_format=CL), w.cuda().contiguous(memory_format=CL)
    flop = 2 * 1 * 6 * 62 * 62 * 512 * 512 * 27
    t_new = _time(lambda: kitchen.try_kernel(xd, wd, b, None, [1, 1, 1]))
    t_ref = _time(lambda: run_ref(ref, xd, wd, b, None, (1, 1, 1)))
    o_new = kitchen.try_kernel(xd, wd, b, None, [1, 1, 1])
    o_ref = run_ref(ref, xd, wd, b, None, (1, 1, 1))
    torch.cuda.synchronize()
    print(f"VAE layer 512->512 3x3x3 on 1x8x64x64: gfx950 {t_new:.3f} ms "
          f"({flop / t_new / 1e9:.0f} TFLOP/s), reference {t_ref:.3f} ms "
          f"({flop / t_ref / 1e9:.0f} TFLOP/s)", flush=True)
    assert torch.allclose(o_new.float(), o_ref.float(), atol=2e-2, rtol=2e-2)
    assert t_new < t_ref
