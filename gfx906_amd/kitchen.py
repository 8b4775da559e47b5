"""gfx950 fp16 conv3d backend for comfy_kitchen's dispatch registry.

Host seam (the reference's ``gfx906_kitchen.py``): comfy_kitchen calls a
registered backend module's ``fp16_conv3d(x, weight, bias, residual, stride)``
and ``fp16_conv3d_out(..., out)``; ``install()`` registers this module as
``"gfx950"`` at the head of the registry's priority list (on a gfx950 device,
or anywhere with ``GFX906_AMD_KITCHEN_FORCE=1`` / the reference's
``GFX906_KITCHEN_FORCE=1``; never without comfy_kitchen or a loadable
kernel).

Work goes to the MI355X implicit-GEMM kernel (``csrc/conv3d_kernel.hip``:
fp16 MFMA with fp32 accumulation over NDHWC tensors, bias and residual fused
into the epilogue) through the extension's ``conv3d(x, w, bias, res, out,
dims, xs, os, rs)`` op, whose argument list is the reference binding's
(hip_conv/conv3d.cpp:30-49). The accept / decline contract is the
reference's (gfx906_kitchen.py:167-238):

* served: fp16 x [N, C, D, H, W] and weight [K, C, T, R, S] on one GPU, VALID
  convolution, strides >= 1, C and K multiples of 8, optional fp16 bias [K]
  and fp16 residual [N, K, Z, P, Q] (``residual`` may be ``out`` itself);
* views are used in place when their channels are innermost and every other
  stride is a multiple of 8 elements (16-byte vector access); x and residual
  in any other layout are converted to channels_last_3d first;
* declined, so that torch's conv runs: everything else, an ``out`` the
  kernel cannot write (strides, a batch stride of 0, memory shared with x,
  weight or bias), and what the kernel's 32-bit offsets and tap table
  cannot hold (over 1024 taps, x or weight spanning 2^31 bytes);
* an ``out`` of the wrong shape, dtype or device is the caller's error
  (ValueError).

:func:`plan` makes that decision and returns either a :class:`ConvCall`
ready for the op or the reason it declines.
"""

from __future__ import annotations

import logging
import os
import sys
from dataclasses import dataclass

import torch

from . import loader

logger = logging.getLogger("gfx906_amd.kitchen")

CL = torch.channels_last_3d
MAX_TAPS = 1024             # taps per filter the kernel's tap walk supports
SPAN_LIMIT = 1 << 31        # bytes one x or weight view may span (32-bit offsets)
VOXEL_LIMIT = (1 << 31) - 256


def is_gfx950() -> bool:
    return loader.is_gfx950()


def load():
    """The extension module (its ``conv3d`` op), or None off a gfx950 device."""
    return loader.load_attention()


# -- layouts ------------------------------------------------------------------------------

def ndhwc_strides(t: torch.Tensor):
    """Element strides (batch, depth, height, width) of a 5-D [N, C, D, H, W]
    view whose channel dim is innermost, when all four are multiples of 8 and
    the spatial ones positive; otherwise None."""
    if t.dim() != 5 or t.stride(1) != 1:
        return None
    sn, _, sd, sh, sw = t.stride()
    if sn < 0 or sd <= 0 or sh <= 0 or sw <= 0:
        return None
    if (sn | sd | sh | sw) % 8:
        return None
    return sn, sd, sh, sw


def packed_strides(shape) -> tuple:
    """ndhwc_strides of a packed channels_last_3d tensor of `shape`."""
    c, d, h, w = shape[1:]
    return c * w * h * d, c * w * h, c * w, c


def may_overlap(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Whether two views can share an element: same storage and intersecting
    [lowest, highest] element offsets."""
    if a.untyped_storage().data_ptr() != b.untyped_storage().data_ptr():
        return False
    lo_a, lo_b = a.storage_offset(), b.storage_offset()
    hi_a = lo_a + sum((n - 1) * st for n, st in zip(a.shape, a.stride()) if n)
    hi_b = lo_b + sum((n - 1) * st for n, st in zip(b.shape, b.stride()) if n)
    return lo_a <= hi_b and lo_b <= hi_a


def _span_bytes(shape, strides) -> int:
    """Bytes from the first element of an NDHWC fp16 view to past its last."""
    n, c, d, h, w = shape
    sn, sd, sh, sw = strides
    return 2 * ((n - 1) * sn + (d - 1) * sd + (h - 1) * sh + (w - 1) * sw + c)


# -- planning -----------------------------------------------------------------------------

@dataclass
class ConvCall:
    """Arguments of one ``conv3d`` op call, already in kernel-readable layouts."""

    x: torch.Tensor
    weight: torch.Tensor
    bias: torch.Tensor | None
    residual: torch.Tensor | None
    out: torch.Tensor
    dims: list      # n, d, h, w, c, k, t, r, s, sd, sh, sw, z, p, q
    xs: list
    os: list
    rs: list

    def run(self, ext) -> torch.Tensor:
        ext.conv3d(self.x, self.weight, self.bias, self.residual, self.out, self.dims,
                   self.xs, self.os, self.rs)
        return self.out


def _output_dims(x, weight, stride):
    """(n, c, d, h, w, k, t, r, s, sd, sh, sw, z, p, q), or a decline reason."""
    if x.dim() != 5 or weight.dim() != 5:
        return "x and weight must be 5-D"
    n, c, d, h, w = x.shape
    k, cw, t, r, s = weight.shape
    sd, sh, sw = (int(v) for v in stride)
    if cw != c:
        return "weight channels differ from x's"
    if min(sd, sh, sw) < 1:
        return "stride below 1"
    if d < t or h < r or w < s:
        return "input smaller than the filter"
    z, p, q = (d - t) // sd + 1, (h - r) // sh + 1, (w - s) // sw + 1
    return n, c, d, h, w, k, t, r, s, sd, sh, sw, z, p, q


def plan(x, weight, bias, residual, stride, out=None):
    """A :class:`ConvCall` for the kernel, or a string naming why it declines."""
    dims = _output_dims(x, weight, stride)
    if isinstance(dims, str):
        return dims
    n, c, d, h, w, k, t, r, s, sd, sh, sw, z, p, q = dims
    o_shape = (n, k, z, p, q)
    if x.dtype != torch.float16 or weight.dtype != torch.float16:
        return "x and weight must be fp16"
    if not x.is_cuda or weight.device != x.device:
        return "x and weight must be on one GPU"
    if min(n, c, k) <= 0 or c % 8 or k % 8:
        return "C and K must be positive multiples of 8"
    if t * r * s > MAX_TAPS or n * z * p * q >= VOXEL_LIMIT:
        return "too many taps or output voxels"
    if bias is not None and (bias.dtype != torch.float16 or tuple(bias.shape) != (k,)):
        return "bias must be fp16 [K]"
    if residual is not None and (residual.dtype != torch.float16
                                 or tuple(residual.shape) != o_shape):
        return "residual must be fp16 [N, K, Z, P, Q]"
    if out is not None and (tuple(out.shape) != o_shape or out.dtype != torch.float16
                            or out.device != x.device):
        raise ValueError("fp16_conv3d: out must be an fp16 [N, K, Z, P, Q] tensor on x's device")

    xs = ndhwc_strides(x)
    if xs is None:
        x = x.contiguous(memory_format=CL)
        xs = packed_strides(x.shape)
    weight = weight.contiguous(memory_format=CL)
    if x.data_ptr() % 16 or weight.data_ptr() % 16:
        return "x or weight not 16-byte aligned"
    if _span_bytes(x.shape, xs) >= SPAN_LIMIT or weight.numel() * 2 >= SPAN_LIMIT:
        return "x or weight spans 2^31 bytes or more"
    if bias is not None:
        bias = bias.to(device=x.device).contiguous()

    if out is None:
        out = torch.empty(o_shape, dtype=torch.float16, device=x.device, memory_format=CL)
        os_ = packed_strides(o_shape)
    else:
        os_ = ndhwc_strides(out)
        if os_ is None or out.data_ptr() % 16:
            return "out is not a channels-innermost, 16-byte aligned view"
        if n > 1 and os_[0] == 0:
            return "out writes every batch to one place"
        # The kernel reads x, weight and bias while writing out; it reads each
        # residual element just before writing the same element of out, so
        # residual may be out itself but not partly overlap it.
        if any(a is not None and may_overlap(out, a) for a in (x, weight, bias)):
            return "out shares memory with an input"
        if residual is not None and residual is not out and may_overlap(out, residual):
            return "out partly overlaps residual"

    rs = (0, 0, 0, 0)
    if residual is not None:
        if residual.device != x.device:
            return "residual on another device"
        rs = ndhwc_strides(residual)
        if rs is None or residual.data_ptr() % 16:
            residual = residual.contiguous(memory_format=CL)
            rs = packed_strides(o_shape)
    return ConvCall(x, weight, bias, residual, out,
                    [n, d, h, w, c, k, t, r, s, sd, sh, sw, z, p, q], list(xs), list(os_),
                    list(rs))


def try_kernel(x, weight, bias, residual, stride, out=None):
    """Run the conv on the kernel and return its output, or None when the
    kernel is unavailable or declines the call."""
    ext = load()
    if ext is None:
        return None
    call = plan(x, weight, bias, residual, stride, out)
    if isinstance(call, str):
        logger.debug("gfx950 conv3d declined: %s", call)
        return None
    return call.run(ext)


# -- comfy_kitchen backend functions ------------------------------------------------------

def fp16_conv3d(x, weight, bias, residual, stride):
    """The conv (+ bias, + residual) as a channels_last_3d tensor: on the
    kernel, or torch's conv when the kernel declines."""
    got = try_kernel(x, weight, bias, residual, stride)
    if got is not None:
        return got
    y = torch.nn.functional.conv3d(x, weight, None if bias is None else bias.to(x.device),
                                   stride=stride).contiguous(memory_format=CL)
    if residual is not None:
        y = y + residual.to(x.device)
    return y


def fp16_conv3d_out(x, weight, bias, residual, stride, out):
    """fp16_conv3d written into ``out`` (computed apart and copied when the
    kernel cannot write ``out`` directly)."""
    if try_kernel(x, weight, bias, residual, stride, out=out) is None:
        out.copy_(fp16_conv3d(x, weight, bias, residual, stride))


# -- registration -------------------------------------------------------------------------

def capabilities():
    """comfy_kitchen constraint objects for the two functions: fp16 5-D x and
    weight, optional fp16 bias and residual, on cuda / hip devices."""
    from comfy_kitchen import constraints as ck

    fp16_5d = ck.ParamConstraint(dtypes=frozenset({torch.float16}),
                                 shape_rules=(ck.ExactDims(5),))
    fp16_or_none = ck.ParamConstraint(dtypes=frozenset({torch.float16, type(None)}))
    conv = ck.FunctionConstraints(
        params={"x": fp16_5d, "weight": fp16_5d, "bias": fp16_or_none,
                "residual": fp16_or_none},
        default_devices=frozenset({"cuda", "hip"}))
    return {"fp16_conv3d": conv, "fp16_conv3d_out": ck.with_out_param(conv)}


def install() -> bool:
    """Register this module as the "gfx950" backend, ahead of every other."""
    forced = any(os.environ.get(v) == "1"
                 for v in ("GFX906_AMD_KITCHEN_FORCE", "GFX906_KITCHEN_FORCE"))
    if not forced and not is_gfx950():
        return False
    try:
        from comfy_kitchen.registry import registry
    except ImportError:
        return False
    if load() is None:
        return False
    registry.register("gfx950", sys.modules[__name__], capabilities())
    order = ["gfx950"] + [name for name in registry._priority if name != "gfx950"]
    registry.set_priority(order)
    logger.info("gfx950 conv3d backend registered (priority: %s)", order)
    return True
