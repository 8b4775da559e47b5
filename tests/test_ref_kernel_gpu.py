"""The reference's own kernel, built unmodified for gfx950 into oracle/_ref/, as a
second checker.

It pins the oracle to the reference's actual behaviour: on the shapes of the
reference's own checks (test_variants.py:78-81) its output agrees with
oracle.attention.sdpa_math_fp32 within the reference's own bar, max-abs < 1e-2
(test.py:19), and with the gfx950 kernel within the same bar. It is also
timed beside the gfx950 kernel on the same GPU at the reference's benchmark
shapes (test_variants.py:88-94: B=1, H=8, S=4096, D=64/128) and must be
slower. Skipped when oracle/_ref was not built (no /root/reference at build
time).
"""

import ctypes
import os

import pytest
import torch

import gfx906_amd
from oracle.attention import error_stats, make_inputs, sdpa_math_fp32

pytestmark = pytest.mark.gpu

REF_LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle",
                       "_ref", "libref_attn.so")


@pytest.fixture(scope="module")
def ref():
    if not os.path.isfile(REF_LIB):
        pytest.skip("oracle/_ref/libref_attn.so not built")
    lib = ctypes.CDLL(REF_LIB)
    lib.launch.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 5 + [ctypes.c_float,
                                                                         ctypes.c_void_p]
    lib.launch.restype = None
    return lib


def run_ref(lib, q, k, v, scale):
    B, H, Sq, D = q.shape
    o = torch.zeros_like(q)
    lib.launch(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H, Sq, k.shape[2], D,
               float(scale), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return o


@pytest.mark.parametrize("Sq,Skv,D", [(256, 256, 64), (100, 300, 64), (256, 256, 128),
                                      (77, 411, 128), (512, 512, 32), (512, 512, 512)])
def test_reference_kernel_agrees_with_oracle(ref, Sq, Skv, D):
    q, k, v = make_inputs(2, 4, Sq, Skv, D, seed=Sq + Skv + D)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    o_ref = run_ref(ref, qd, kd, vd, 0.125)
    o_new = gfx906_amd.attn(qd, kd, vd, 0.125)
    torch.cuda.synchronize()
    oracle = sdpa_math_fp32(q, k, v, 0.125)
    mx_ref, _ = error_stats(o_ref.float().cpu(), oracle)
    mx_new, _ = error_stats(o_new.float().cpu(), o_ref.float().cpu())
    print(f"Sq{Sq} Skv{Skv} D{D}: reference kernel vs oracle {mx_ref:.2e}, "
          f"gfx950 kernel vs reference kernel {mx_new:.2e}", flush=True)
    assert mx_ref < 1e-2 and mx_new < 1e-2


@pytest.mark.parametrize("D", [64, 128])
def test_faster_than_reference_kernel_on_same_gpu(ref, D):
    q, k, v = (t.cuda() for t in make_inputs(1, 8, 4096, 4096, D, seed=D))

    def timeit(fn, n=5):
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        best = float("inf")
        for _ in range(n):
            a.record()
            fn()
            b.record()
            b.synchronize()
            best = min(best, a.elapsed_time(b))
        return best

    o = torch.empty_like(q)
    stream = torch.cuda.current_stream().cuda_stream

    def ref_call():
        ref.launch(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), 1, 8, 4096, 4096, D,
                   0.125, stream)

    t_ref = timeit(ref_call)
    t_new = timeit(lambda: gfx906_amd.attn(q, k, v, 0.125))
    fl = gfx906_amd.flops(1, 8, 4096, 4096, D)
    print(f"D={D} B1 H8 S4096: reference kernel {t_ref:.3f} ms ({fl / t_ref / 1e9:.1f} TFLOP/s), "
          f"gfx950 kernel {t_new:.3f} ms ({fl / t_new / 1e9:.1f} TFLOP/s), "
          f"speed-up {t_ref / t_new:.1f}x", flush=True)
    assert t_new < t_ref
