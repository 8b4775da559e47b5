"""gfx950 fp16 conv3d backend for comfy_kitchen's dispatch registry.

Counterpart of the reference's ``gfx906_kitchen.py`` (its public functions and
their caller contract: ``load``, ``fp16_conv3d``, ``fp16_conv3d_out``,
``install``, and ``_conv3d_into`` returning ``None`` when the call is not the
kernel's to serve, gfx906_kitchen.py:85-299), on the MI355X implicit-GEMM
kernel (``gfx906_amd/csrc/conv3d_kernel.hip``: matrix-core fp16 MFMA with fp32
accumulation over NDHWC tensors, fused bias and residual).

* Served: fp16 x [N, C, D, H, W] and weight [K, C, T, R, S] on one GPU, VALID
  convolution with strides >= 1, C and K multiples of 8, optional fp16 bias
  [K] and residual [N, K, Z, P, Q] (gfx906_kitchen.py:178-186). x is read in
  place when it is NDHWC-indexable (channel stride 1, other strides multiples
  of 8); otherwise it is converted to channels_last_3d. The result is a packed
  channels_last_3d tensor, or ``out`` when given.
* Declined (torch's conv runs instead in ``fp16_conv3d``): everything else,
  plus what this kernel's 32-bit offsets and tap table cannot hold (more than
  1024 taps, x or weight spanning 2^31 bytes or more).
* ``install()`` registers the backend as ``"gfx950"`` with top priority; it is
  a no-op off a gfx950 device unless ``GFX906_AMD_KITCHEN_FORCE=1`` (or the
  reference's ``GFX906_KITCHEN_FORCE=1``) and when comfy_kitchen is absent.
"""

from __future__ import annotations

import logging
import os
import sys

import torch

from . import loader

logger = logging.getLogger("gfx906_amd.kitchen")

_CL = torch.channels_last_3d
_MAX_TAPS = 1024
_SPAN_LIMIT = 1 << 31
_M_LIMIT = (1 << 31) - 256


def is_gfx950() -> bool:
    return loader.is_gfx950()


def load():
    """The extension module (its ``conv3d`` op), or None off a gfx950 device."""
    return loader.load_attention()


# -- layouts --------------------------------------------------------------------------------

def _ndhwc_strides(t: torch.Tensor):
    """(sn, sd, sh, sw) element strides of a 5-D [N, C, D, H, W] view whose channels are
    innermost, or None. Spatial strides must be positive and every stride a multiple of 8
    (16-byte vector loads)."""
    if t.dim() != 5:
        return None
    sn, sc, sd, sh, sw = t.stride()
    if sc != 1 or sn < 0 or min(sd, sh, sw) <= 0:
        return None
    st = (sn, sd, sh, sw)
    return st if all(s % 8 == 0 for s in st) else None


def _out_strides(t: torch.Tensor):
    """Same rule for an [N, K, Z, P, Q] output or residual (K innermost)."""
    return _ndhwc_strides(t)


def _packed_strides(shape) -> tuple:
    """(sn, sd, sh, sw) of a packed channels_last_3d tensor of `shape` [N, C, D, H, W]."""
    _, c, d, h, w = shape
    return (d * h * w * c, h * w * c, w * c, c)


def _tensors_overlap(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Whether the element ranges of two tensors may share memory (same storage and
    intersecting [first, last] extents)."""
    if a.untyped_storage().data_ptr() != b.untyped_storage().data_ptr():
        return False

    def extent(t):
        lo = t.storage_offset()
        hi = lo + sum((n - 1) * s for n, s in zip(t.shape, t.stride()) if n > 0)
        return lo, hi

    (a0, a1), (b0, b1) = extent(a), extent(b)
    return a0 <= b1 and b0 <= a1


def _span_bytes(shape, strides) -> int:
    """Bytes from the first to one past the last element of an NDHWC fp16 view."""
    n, c, d, h, w = shape
    sn, sd, sh, sw = strides
    return ((n - 1) * sn + (d - 1) * sd + (h - 1) * sh + (w - 1) * sw + c) * 2


# -- backend --------------------------------------------------------------------------------

def _conv3d_into(x, weight, bias, residual, stride, out=None):
    """The kernel's result tensor, or None when the call is not ours to serve."""
    ext = load()
    if ext is None:
        return None
    if x.dim() != 5 or weight.dim() != 5:
        return None
    n, c, d, h, w = x.shape
    k, cw, t, r, s = weight.shape
    sd, sh, sw = (int(v) for v in stride)
    if min(sd, sh, sw) < 1 or d < t or h < r or w < s:
        return None
    z, p, q = (d - t) // sd + 1, (h - r) // sh + 1, (w - s) // sw + 1
    M = n * z * p * q
    if not (x.dtype == torch.float16 and weight.dtype == torch.float16 and x.is_cuda
            and weight.device == x.device and cw == c and c % 8 == 0 and k % 8 == 0
            and min(n, c, k) > 0 and M < _M_LIMIT and t * r * s <= _MAX_TAPS
            and (bias is None or (bias.dtype == torch.float16 and bias.shape == (k,)))
            and (residual is None or (residual.dtype == torch.float16
                                      and residual.shape == (n, k, z, p, q)))):
        return None
    xs = _ndhwc_strides(x)
    if xs is None:
        x = x.contiguous(memory_format=_CL)
        xs = _packed_strides(x.shape)
    weight = weight.contiguous(memory_format=_CL)
    if (x.data_ptr() % 16 or weight.data_ptr() % 16
            or _span_bytes(x.shape, xs) >= _SPAN_LIMIT
            or k * c * t * r * s * 2 >= _SPAN_LIMIT):
        return None
    if bias is not None:
        bias = bias.to(device=x.device).contiguous()

    if out is None:
        out = torch.empty((n, k, z, p, q), dtype=torch.float16, device=x.device,
                          memory_format=_CL)
        ostr = _packed_strides(out.shape)
    else:
        if out.shape != (n, k, z, p, q) or out.dtype != torch.float16 or out.device != x.device:
            raise ValueError("fp16_conv3d: out must be an fp16 [N, K, Z, P, Q] tensor on x's device")
        ostr = _out_strides(out)
        if ostr is None or out.data_ptr() % 16:
            return None
        if n > 1 and ostr[0] == 0:  # batches written onto each other
            return None
        # Reads of x, weight or bias would race the writes; residual is read and
        # written element by element by the same lane, so residual is out is fine.
        if any(o is not None and _tensors_overlap(out, o) for o in (x, weight, bias)):
            return None
        if residual is not None and residual is not out and _tensors_overlap(out, residual):
            return None

    if residual is None:
        rstr = (0, 0, 0, 0)
    else:
        if residual.device != x.device:
            return None
        rstr = _out_strides(residual)
        if rstr is None or residual.data_ptr() % 16:
            residual = residual.contiguous(memory_format=_CL)
            rstr = _packed_strides(residual.shape)

    ext.conv3d(x, weight, bias, residual, out, [n, d, h, w, c, k, t, r, s, sd, sh, sw, z, p, q],
               list(xs), list(ostr), list(rstr))
    return out


def fp16_conv3d(x, weight, bias, residual, stride):
    """comfy_kitchen fp16_conv3d entry: the kernel, or torch's conv when it declines."""
    out = _conv3d_into(x, weight, bias, residual, stride)
    if out is not None:
        return out
    bias = None if bias is None else bias.to(device=x.device)
    res = torch.nn.functional.conv3d(x, weight, bias, stride=stride).contiguous(memory_format=_CL)
    return res if residual is None else res + residual.to(device=x.device)


def fp16_conv3d_out(x, weight, bias, residual, stride, out):
    """fp16_conv3d into ``out``; computed then copied when out is not kernel-writable."""
    if _conv3d_into(x, weight, bias, residual, stride, out=out) is not None:
        return
    out.copy_(fp16_conv3d(x, weight, bias, residual, stride))


# -- registration --------------------------------------------------------------------------

def _capabilities():
    from comfy_kitchen.constraints import (ExactDims, FunctionConstraints, ParamConstraint,
                                           with_out_param)

    devices = frozenset({"cuda", "hip"})
    fp16_5d = ParamConstraint(dtypes=frozenset({torch.float16}), shape_rules=(ExactDims(5),))
    fp16_opt = ParamConstraint(dtypes=frozenset({torch.float16, type(None)}))
    conv = FunctionConstraints(
        params={"x": fp16_5d, "weight": fp16_5d, "bias": fp16_opt, "residual": fp16_opt},
        default_devices=devices)
    return {"fp16_conv3d": conv, "fp16_conv3d_out": with_out_param(conv)}


def install() -> bool:
    """Register the backend as "gfx950" first in comfy_kitchen's priority list."""
    forced = any(os.environ.get(v) == "1"
                 for v in ("GFX906_AMD_KITCHEN_FORCE", "GFX906_KITCHEN_FORCE"))
    if not (is_gfx950() or forced):
        return False
    try:
        from comfy_kitchen.registry import registry
    except ImportError:
        return False
    if load() is None:
        return False
    registry.register("gfx950", sys.modules[__name__], _capabilities())
    registry.set_priority(["gfx950"] + [b for b in registry._priority if b != "gfx950"])
    logger.info("gfx950 conv3d backend registered (priority: %s)", registry._priority)
    return True
