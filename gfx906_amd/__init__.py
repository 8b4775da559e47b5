"""MI355X (gfx950) flash-attention forward behind the reference's
``attn(q, k, v, scale)`` operator.

``attn`` runs the hand-written HIP kernel on fp16 or bf16 ``[B, H, S, D]`` CUDA
tensors (D <= 64 and a multiple of 8, or 128, or 512; Sq may differ from Skv;
strided views with a contiguous head dim are read in place) and returns a new
tensor of the input dtype, or writes ``out``. It raises if the HIP libraries
are not built or the inputs are not accepted; there is no fallback
implementation.
"""

from .loader import (KERNEL_LIB, EXT_LIB, NotBuiltError, capi, extension,  # noqa: F401
                     is_gfx950, load_attention)


def attn(q, k, v, scale, out=None):
    """o = softmax(scale * q k^T) v for [B,H,Sq,D] q and [B,H,Skv,D] k, v (fp16 or
    bf16), into a new tensor or into ``out`` (a [B,H,Sq,D] view, e.g. of a
    [B,Sq,H,D] buffer)."""
    return extension().attn(q, k, v, float(scale), out)


def flops(B, H, Sq, Skv, D):
    """Algorithmic FLOPs of one forward: 4*B*H*Sq*Skv*D (flops_probe.py:18)."""
    return 4 * B * H * Sq * Skv * D
