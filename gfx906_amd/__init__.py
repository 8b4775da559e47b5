"""MI355X (gfx950) flash-attention forward behind the reference's
``attn(q, k, v, scale)`` operator.

``attn`` runs the hand-written HIP kernel on fp16 ``[B, H, S, D]`` CUDA tensors
(D <= 64 and a multiple of 8, or 128, or 512; Sq may differ from Skv) and
returns a new fp16 tensor. It raises if the HIP libraries are not built or
the inputs are not accepted; there is no fallback implementation.
"""

from .loader import (KERNEL_LIB, EXT_LIB, NotBuiltError, capi, extension,  # noqa: F401
                     is_gfx950, load_attention)


def attn(q, k, v, scale):
    """o = softmax(scale * q k^T) v for fp16 [B,H,Sq,D] q and [B,H,Skv,D] k, v."""
    return extension().attn(q, k, v, float(scale))


def flops(B, H, Sq, Skv, D):
    """Algorithmic FLOPs of one forward: 4*B*H*Sq*Skv*D (flops_probe.py:18)."""
    return 4 * B * H * Sq * Skv * D
