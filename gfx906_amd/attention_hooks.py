"""Send a host application's attention calls to the gfx950 kernel.

Host seams (the ComfyUI ones the reference hooks, deploy/gfx906_attention.py):

* ``comfy.ldm.modules.attention.optimized_attention.container_function``:
  called with containers of [B, H, S, D] q/k/v (``peek()`` looks, ``take()``
  hands the tensor over) and ``(heads, mask, attn_precision, skip_reshape,
  skip_output_reshape, **kwargs)``; returns [B, S, H*D], or [B, H, S, D] with
  ``skip_output_reshape``. ``install()`` fills this slot once, on gfx950 only,
  and never replaces a function someone else put there.
* ``comfy.ldm.modules.diffusionmodules.model.vae_attention``: a factory
  returning the VAE mid-block attention f(q, k, v) on [b, c, h, w]. With
  ``GFX906_AMD_VAE=1`` (or the reference's ``SEEDVR2_GFX906_VAE=1``) the
  factory is wrapped so that, when it picks the slice (``normal_attention``)
  or PyTorch path, c = 512 calls run on the kernel as one [b, 1, h*w, c]
  attention; any other choice is returned untouched.

What runs on the kernel is the reference's eligibility rule
(deploy/gfx906_attention.py:38-49): no mask and no GQA, CUDA fp16/bf16 4-D
tensors with equal B, H and D, ``k.shape == v.shape``, H equal to ``heads``,
D in {128, 512} or D <= 64 and a multiple of 8, and q/k/v already in
[B, H, S, D] (``skip_reshape``). :func:`decline_reason` names the rule a call
fails. Everything declined, and any call the kernel raises on, goes to the
host's own function with the original arguments.

Differences from the reference, by design: bf16 runs natively (no fp16
round trip); the [B, S, H*D] result is written by the kernel through a
transposed view of the output buffer, and the VAE result through a
token-contiguous view of the [b, c, h, w] output, so no layout copies
follow; a kernel error on the DiT path also falls back (the reference only
does so for the VAE). ``GFX906_AMD_LOG_SHAPES=1`` (or
``SEEDVR2_GFX906_LOG_SHAPES=1``) logs each new kernel shape once.

Nothing here imports the host application until ``install()`` runs.
"""

from __future__ import annotations

import logging
import os

import torch

from . import loader

logger = logging.getLogger("gfx906_amd")

KERNEL_DTYPES = (torch.float16, torch.bfloat16)
VAE_CHANNELS = 512


def _env_on(*names) -> bool:
    return any(os.environ.get(n) == "1" for n in names)


def head_dim_supported(d: int) -> bool:
    """Head dims the kernel accepts: <= 64 and a multiple of 8, or 128, or 512."""
    return d in (128, 512) or (0 < d <= 64 and d % 8 == 0)


def decline_reason(qt, kt, vt, heads, mask, kwargs):
    """Why a [B, H, S, D] call cannot run on the kernel, or None if it can."""
    if mask is not None:
        return "mask"
    if kwargs.get("enable_gqa"):
        return "grouped-query attention"
    if not qt.is_cuda or qt.dtype not in KERNEL_DTYPES:
        return "not a CUDA fp16/bf16 tensor"
    if qt.ndim != 4 or kt.ndim != 4:
        return "not 4-D"
    if kt.shape != vt.shape:
        return "k and v shapes differ"
    (b, h, _, d), (bk, hk, _, dk) = qt.shape, kt.shape
    if (b, h, d) != (bk, hk, dk):
        return "q and k disagree on batch, heads or head dim"
    if h != heads:
        return "head count differs from `heads`"
    if not head_dim_supported(d):
        return f"head dim {d}"
    return None


def eligible(qt, kt, vt, heads, mask, kwargs) -> bool:
    return decline_reason(qt, kt, vt, heads, mask, kwargs) is None


class DitRouter:
    """The ``container_function``: kernel for eligible calls, the wrapped
    ``optimized_attention`` (``stock``) for the rest."""

    def __init__(self):
        self.stock = None
        self.log_shapes = _env_on("GFX906_AMD_LOG_SHAPES", "SEEDVR2_GFX906_LOG_SHAPES")
        self._logged = set()

    def __call__(self, q, k, v, heads, mask=None, attn_precision=None, skip_reshape=False,
                 skip_output_reshape=False, **kwargs):
        qt, kt, vt = q.peek(), k.peek(), v.peek()
        mod = None
        if skip_reshape and eligible(qt, kt, vt, heads, mask, kwargs):
            mod = loader.load_attention()
        qt, kt, vt = q.take(), k.take(), v.take()
        if mod is not None:
            try:
                return self._on_kernel(mod, qt, kt, vt, kwargs.get("scale"), skip_output_reshape)
            except RuntimeError as exc:
                logger.warning("gfx950 attention failed on %s (%s); using the stock path",
                               tuple(qt.shape), exc)
        return self.stock(qt, kt, vt, heads, mask=mask, attn_precision=attn_precision,
                          skip_reshape=skip_reshape, skip_output_reshape=skip_output_reshape,
                          **kwargs)

    def _on_kernel(self, mod, qt, kt, vt, scale, bhsd_out):
        if self.log_shapes and qt.shape not in self._logged:
            self._logged.add(qt.shape)
            logger.info("gfx950 attention: %s %s", tuple(qt.shape), qt.dtype)
        if scale is None:
            scale = qt.shape[-1] ** -0.5  # SDPA's default
        if bhsd_out:
            return mod.attn(qt, kt, vt, scale)
        b, h, s, d = qt.shape
        tokens = torch.empty((b, s, h, d), dtype=qt.dtype, device=qt.device)
        mod.attn(qt, kt, vt, scale, out=tokens.transpose(1, 2))  # written as [B, S, H, D]
        return tokens.view(b, s, h * d)


def _token_view(x):
    """[b, c, h, w] -> [b, 1, h*w, c] view (sequence stride 1, channel stride
    h*w). The op reads and writes such views in place, or copies them where
    that is faster (h*w > 6400)."""
    b, c, h, w = x.shape
    return x.reshape(b, c, h * w).transpose(1, 2).unsqueeze(1)


def vae_attn(q, k, v, fallback):
    """VAE mid-block attention on [b, c, h, w] tensors, c = 512: one
    [b, 1, h*w, c] attention with scale c**-0.5 on the kernel. ``fallback``
    (the function the host's factory chose) serves every other call and any
    call the kernel raises on."""
    mod = None
    if (q.is_cuda and q.dtype in KERNEL_DTYPES and q.dim() == 4
            and q.shape == k.shape == v.shape and q.shape[1] == VAE_CHANNELS):
        mod = loader.load_attention()
    if mod is None:
        return fallback(q, k, v)
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    try:
        mod.attn(_token_view(q), _token_view(k), _token_view(v), q.shape[1] ** -0.5,
                 out=_token_view(out))
    except Exception as exc:  # noqa: BLE001 - a decode must not fail on the fast path
        logger.warning("gfx950 VAE attention failed (%s); using %s", exc,
                       getattr(fallback, "__name__", fallback))
        return fallback(q, k, v)
    return out


class VaeRouter:
    """Wraps the host's ``vae_attention`` factory (``model.vae_attention``)."""

    def __init__(self):
        self.model = None

    def attach(self, model) -> bool:
        if self.model is not None:
            return False
        self.model = model
        routed = (model.normal_attention, getattr(model, "pytorch_attention", None))
        choose = model.vae_attention

        def vae_attention():
            chosen = choose()
            if not any(chosen is f for f in routed if f is not None):
                return chosen  # e.g. xformers: not ours to replace
            return lambda q, k, v: vae_attn(q, k, v, chosen)

        model.vae_attention = vae_attention
        return True


dit = DitRouter()
vae = VaeRouter()
container_attn = dit  # the callable installed as container_function


def install_vae_hook() -> None:
    """Wrap ``vae_attention()`` so its slice / PyTorch choices run on the kernel."""
    try:
        from comfy.ldm.modules.diffusionmodules import model
    except Exception as exc:  # noqa: BLE001 - host application not importable
        logger.warning("gfx950 VAE attention hook skipped: %s", exc)
        return
    if vae.attach(model):
        logger.info("gfx950 attention installed (VAE mid-block, D=512)")


def install() -> None:
    """Fill ``optimized_attention.container_function`` once; nothing off gfx950."""
    if not loader.is_gfx950():
        return
    try:
        from comfy.ldm.modules import attention as host
    except Exception as exc:  # noqa: BLE001 - host application not importable
        logger.warning("gfx950 attention hook skipped: %s", exc)
        return
    slot_owner = host.optimized_attention
    if dit.stock is slot_owner or not hasattr(slot_owner, "container_function"):
        return
    if slot_owner.container_function is not None:
        logger.warning("optimized_attention.container_function is taken; "
                       "gfx950 attention not installed")
        return
    dit.stock = slot_owner
    slot_owner.container_function = container_attn
    logger.info("gfx950 attention installed (DiT)")
    if _env_on("GFX906_AMD_VAE", "SEEDVR2_GFX906_VAE"):
        install_vae_hook()
