"""The SDPA hook layer on the GPU: DiT container calls ([B, H, S, D] in, [B, S, H*D]
out, fp16 and bf16) and the VAE mid-block call ([b, 512, h, w]) through the real
kernel, against torch SDPA MATH in fp32 on the CPU."""

import pytest
import torch

from gfx906_amd import attention_hooks as hooks
from gfx906_amd import loader
from oracle.attention import MAX_ABS_TOL, MEAN_ABS_TOL, error_stats, make_inputs, sdpa_math_fp32

pytestmark = pytest.mark.gpu


class Box:
    def __init__(self, t):
        self.t = t

    def peek(self):
        return self.t

    def take(self):
        return self.t


def setup_module():
    loader._attempted = False
    assert loader.load_attention() is not None, "kernel must load on the MI355X"


@pytest.mark.parametrize("dtype,D", [(torch.float16, 128), (torch.bfloat16, 128),
                                     (torch.float16, 64)])
def test_dit_container_call(dtype, D):
    q, k, v = make_inputs(2, 6, 333, 333, D, seed=D)
    qd, kd, vd = (t.to("cuda", dtype) for t in (q, k, v))
    with pytest.MonkeyPatch.context() as mp:
        mp.setattr(hooks.dit, "stock", None)  # the kernel path must be taken
        out = hooks.container_attn(Box(qd), Box(kd), Box(vd), 6, skip_reshape=True)
    torch.cuda.synchronize()
    assert out.dtype == dtype and out.shape == (2, 333, 6 * D)
    ref = sdpa_math_fp32(qd.cpu(), kd.cpu(), vd.cpu(), D ** -0.5)
    ref = ref.transpose(1, 2).reshape(2, 333, 6 * D)
    mx, mn = error_stats(out.float().cpu(), ref)
    tol = (MAX_ABS_TOL, MEAN_ABS_TOL) if dtype == torch.float16 else (2e-2, 2e-3)
    assert mx <= tol[0] and mn <= tol[1], (mx, mn)


def test_vae_call():
    g = torch.Generator().manual_seed(3)
    x = [(torch.randn(1, 512, 12, 20, generator=g) * 0.5).half() for _ in range(3)]

    def fallback(q, k, v):
        raise AssertionError("fallback must not run")

    out = hooks.vae_attn(*(t.cuda() for t in x), fallback)
    torch.cuda.synchronize()
    assert out.shape == (1, 512, 12, 20)
    tok = [t.reshape(1, 512, 240).transpose(1, 2).unsqueeze(1) for t in x]
    ref = sdpa_math_fp32(*tok, 512 ** -0.5).squeeze(1).transpose(1, 2).reshape(1, 512, 12, 20)
    mx, mn = error_stats(out.float().cpu(), ref)
    assert mx <= MAX_ABS_TOL and mn <= MEAN_ABS_TOL, (mx, mn)
