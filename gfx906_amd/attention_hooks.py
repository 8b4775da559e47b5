"""Route a host application's scaled-dot-product attention through the gfx950 kernel.

Counterpart of the reference's ComfyUI hook layer (deploy/gfx906_attention.py:1-163),
with the same caller contract:

* :func:`install` sets ``optimized_attention.container_function`` (the seam
  ``comfy.ldm.modules.attention`` keeps for containerised q/k/v) once, on a
  gfx950 device only (reference ``install``, :140-162). An already-set
  container function is left alone.
* :func:`container_attn` takes the kernel path for eligible calls (:func:`eligible`,
  reference :38-49: no mask or GQA, fp16/bf16 CUDA 4-D tensors with equal B, H
  and D, ``k.shape == v.shape``, ``H == heads``, D in {128, 512} or D <= 64 and a
  multiple of 8, and ``skip_reshape=True``) and returns ``[B, S, H*D]`` unless
  ``skip_output_reshape`` (:76-79). Where the reference casts bf16 to fp16 and
  back around its kernel (:71-75), bf16 runs natively here, and the
  ``[B, S, H*D]`` result is written by the kernel in that layout (no transpose
  copy). Anything else goes to the stock callable unchanged (:58-62).
* :func:`vae_attn` serves the VAE mid-block attention (``[b, c, h, w]``,
  c = 512) as one ``[b, 1, h*w, c]`` attention and falls back to the
  function the factory selected if the kernel raises (:82-111);
  :func:`install_vae_hook` wraps ``vae_attention()`` so that only its slice
  and PyTorch paths are intercepted (:114-137). It is installed when
  ``GFX906_AMD_VAE=1`` (or the reference's ``SEEDVR2_GFX906_VAE=1``).
* ``GFX906_AMD_LOG_SHAPES=1`` (or ``SEEDVR2_GFX906_LOG_SHAPES=1``) logs each new
  shape once (:30-31, :63-65).

The host application is imported lazily; nothing here imports it at module load.
"""

from __future__ import annotations

import logging
import os

import torch

from . import loader

logger = logging.getLogger("gfx906_amd")


def _flag(*names):
    return any(os.environ.get(n) == "1" for n in names)


_LOG_SHAPES = _flag("GFX906_AMD_LOG_SHAPES", "SEEDVR2_GFX906_LOG_SHAPES")
_VAE_HOOK = _flag("GFX906_AMD_VAE", "SEEDVR2_GFX906_VAE")
_seen_shapes: set = set()

_stock_attention = None         # the wrapped optimized_attention (fallback)
_stock_normal_attention = None  # diffusionmodules.model.normal_attention, once hooked


def head_dim_supported(d: int) -> bool:
    """Head dims the kernel accepts: <= 64 and a multiple of 8, or 128, or 512."""
    return d in (128, 512) or (0 < d <= 64 and d % 8 == 0)


def eligible(qt, kt, vt, heads, mask, kwargs) -> bool:
    """Whether a [B, H, S, D] call can take the kernel path."""
    if mask is not None or kwargs.get("enable_gqa"):
        return False
    if qt.dtype not in (torch.float16, torch.bfloat16) or not qt.is_cuda:
        return False
    if qt.ndim != 4 or kt.ndim != 4 or kt.shape != vt.shape:
        return False
    if (qt.shape[0] != kt.shape[0] or qt.shape[1] != kt.shape[1]
            or qt.shape[3] != kt.shape[3] or qt.shape[1] != heads):
        return False
    return head_dim_supported(qt.shape[3])


def container_attn(q, k, v, heads, mask=None, attn_precision=None, skip_reshape=False,
                   skip_output_reshape=False, **kwargs):
    """``container_function`` for ``optimized_attention``: q/k/v are containers
    with ``peek()`` (look without releasing) and ``take()`` (release)."""
    qt, kt, vt = q.peek(), k.peek(), v.peek()
    mod = None
    if skip_reshape and eligible(qt, kt, vt, heads, mask, kwargs):
        mod = loader.load_attention()
    if mod is None:
        return _stock_attention(q.take(), k.take(), v.take(), heads, mask=mask,
                                attn_precision=attn_precision, skip_reshape=skip_reshape,
                                skip_output_reshape=skip_output_reshape, **kwargs)
    if _LOG_SHAPES and tuple(qt.shape) not in _seen_shapes:
        _seen_shapes.add(tuple(qt.shape))
        logger.info("gfx950 attention: %s %s", tuple(qt.shape), qt.dtype)
    qt, kt, vt = q.take(), k.take(), v.take()
    scale = kwargs.get("scale")
    if scale is None:
        scale = qt.shape[-1] ** -0.5  # SDPA's default
    if skip_output_reshape:
        return mod.attn(qt, kt, vt, scale)
    b, h, s, d = qt.shape
    out = torch.empty((b, s, h, d), dtype=qt.dtype, device=qt.device)
    mod.attn(qt, kt, vt, scale, out=out.transpose(1, 2))
    return out.view(b, s, h * d)


def vae_attn(q, k, v, fallback):
    """Drop-in for the VAE ``normal_attention`` ([b, c, h, w] -> same shape).

    Eligible calls (CUDA fp16/bf16, c == 512) run as one [b, 1, h*w, c]
    attention with scale c**-0.5; anything else, or a kernel error, uses
    ``fallback``, the function the factory selected.
    """
    mod = None
    if (q.is_cuda and q.dtype in (torch.float16, torch.bfloat16) and q.dim() == 4
            and q.shape == k.shape == v.shape and q.shape[1] == 512):
        mod = loader.load_attention()
    if mod is None:
        return fallback(q, k, v)
    b, c, h, w = q.shape

    def tokens(x):  # [b, c, h, w] -> [b, 1, h*w, c]: a token-contiguous view (sequence
        # stride 1, channel stride h*w); the op reads and writes such views in place,
        # or through copies where that is faster (h*w > 8192)
        return x.reshape(b, c, h * w).transpose(1, 2).unsqueeze(1)

    out = torch.empty((b, c, h, w), dtype=q.dtype, device=q.device)
    try:
        mod.attn(tokens(q), tokens(k), tokens(v), c ** -0.5, out=tokens(out))
    except Exception:  # noqa: BLE001 - a VAE decode must not fail on the fast path
        logger.warning("gfx950 VAE attention failed; using %s",
                       getattr(fallback, "__name__", fallback))
        return fallback(q, k, v)
    return out


def install_vae_hook() -> None:
    """Wrap ``vae_attention()`` so that its slice / PyTorch choices go to the kernel."""
    global _stock_normal_attention
    try:
        from comfy.ldm.modules.diffusionmodules import model as _model
    except Exception as exc:  # noqa: BLE001 - host application not importable
        logger.warning("gfx950 VAE attention hook skipped: %s", exc)
        return
    if _stock_normal_attention is not None:
        return
    _stock_normal_attention = _model.normal_attention
    intercepted = {_model.normal_attention, getattr(_model, "pytorch_attention", None)}
    orig_factory = _model.vae_attention

    def factory():
        fn = orig_factory()
        if fn not in intercepted:
            return fn  # another backend was selected: leave it alone
        return lambda q, k, v: vae_attn(q, k, v, fn)

    _model.vae_attention = factory
    logger.info("gfx950 attention installed (VAE mid-block, D=512)")


def install() -> None:
    """Hook ``optimized_attention.container_function`` once. No-op off gfx950."""
    global _stock_attention
    if not loader.is_gfx950():
        return
    try:
        from comfy.ldm.modules import attention as _attn
    except Exception as exc:  # noqa: BLE001 - host application not importable
        logger.warning("gfx950 attention hook skipped: %s", exc)
        return
    opt = _attn.optimized_attention
    if _stock_attention is opt or not hasattr(opt, "container_function"):
        return
    if opt.container_function is not None:
        logger.warning("optimized_attention.container_function already set; "
                       "gfx950 attention hook not installed")
        return
    _stock_attention = opt
    opt.container_function = container_attn
    logger.info("gfx950 attention installed (DiT)")
    if _VAE_HOOK:
        install_vae_hook()
