"""Loading of the built gfx950 attention libraries.

:func:`extension` returns the torch binding module (``attn(q, k, v, scale)``)
and raises if it has not been built, so nothing silently falls back to
another implementation. :func:`load_attention` keeps the reference loader's
caller contract (deploy/gfx906_attn.py:28-88): on a gfx950 device it builds
what is missing or out of date (the kernel library with hipcc, once, with a
failure marker that stops retries; the binding with
``torch.utils.cpp_extension.load``) and returns the module; off gfx950, or
when a build or load fails, it returns ``None`` so a hook layer keeps its
stock attention path. The first outcome is cached.
"""

from __future__ import annotations

import ctypes
import importlib.util
import logging
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB = PKG / "lib"
KERNEL_LIB = LIB / "libgfx906_amd_attn.so"
EXT_NAME = "gfx906_amd_attn_ext"
EXT_LIB = LIB / f"{EXT_NAME}.so"

logger = logging.getLogger("gfx906_amd")

_ext = None
_attempted = False
_module = None


class NotBuiltError(ImportError):
    """The HIP libraries are missing: run ``python -m gfx906_amd.build``."""


def extension():
    """The torch extension module; raises NotBuiltError if it is not built."""
    global _ext
    if _ext is not None:
        return _ext
    if not EXT_LIB.is_file() or not KERNEL_LIB.is_file():
        raise NotBuiltError(
            f"gfx950 attention libraries not built ({EXT_LIB}); run python -m gfx906_amd.build")
    import torch  # noqa: F401  -- the extension links against torch's libraries

    if EXT_NAME in sys.modules:
        _ext = sys.modules[EXT_NAME]
        return _ext
    spec = importlib.util.spec_from_file_location(EXT_NAME, EXT_LIB)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    sys.modules[EXT_NAME] = mod
    _ext = mod
    return mod


def capi() -> ctypes.CDLL:
    """ctypes handle on the C-ABI library (symbols of include/gfx906_amd_attn.h)."""
    if not KERNEL_LIB.is_file():
        raise NotBuiltError(f"{KERNEL_LIB} not built; run python -m gfx906_amd.build")
    lib = ctypes.CDLL(str(KERNEL_LIB))
    args = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 5 + [ctypes.c_float, ctypes.c_void_p]
    lib.launch.argtypes = args
    lib.launch.restype = None
    lib.attn_fwd.argtypes = args
    lib.attn_fwd.restype = ctypes.c_int
    strides = ctypes.POINTER(ctypes.c_longlong)
    lib.attn_fwd_ex.argtypes = args + [ctypes.c_int] + [strides] * 4
    lib.attn_fwd_ex.restype = ctypes.c_int
    lib.attn_fwd_split.argtypes = lib.attn_fwd_ex.argtypes + [ctypes.c_void_p, ctypes.c_size_t]
    lib.attn_fwd_split.restype = ctypes.c_int
    lib.attn_split_workspace_bytes.argtypes = [ctypes.c_int] * 5
    lib.attn_split_workspace_bytes.restype = ctypes.c_size_t
    lib.attn_fwd_split_static.argtypes = lib.attn_fwd_ex.argtypes
    lib.attn_fwd_split_static.restype = ctypes.c_int
    lib.attn_split_scratch_capacity.argtypes = []
    lib.attn_split_scratch_capacity.restype = ctypes.c_size_t
    lib.attn_last_error.argtypes = []
    lib.attn_last_error.restype = ctypes.c_char_p
    return lib


def is_gfx950() -> bool:
    """True when the current device is a gfx950 (MI350/MI355) GPU.

    Counterpart of the reference's arch gate (deploy/gfx906_attn.py:28-37).
    """
    import torch

    if not torch.cuda.is_available():
        return False
    try:
        arch = torch.cuda.get_device_properties(torch.cuda.current_device()).gcnArchName
    except Exception:  # noqa: BLE001 - builds without gcnArchName
        return False
    return arch.startswith("gfx950")


def load_attention():
    """Return the extension module (has ``attn(q, k, v, scale)``) or ``None``.

    ``None`` off gfx950, when the kernel library cannot be built (see
    gfx906_amd.build.ensure_kernel_lib: a failed build is not retried until a
    source changes) or when the binding cannot be built or loaded. The first
    outcome is cached, as in deploy/gfx906_attn.py:62-88.
    """
    global _module, _attempted, _ext
    if _attempted:
        return _module
    _attempted = True
    try:
        if not is_gfx950():
            return None
        from . import build

        if not build.ensure_kernel_lib():
            return None
        if build.extension_stale():
            mod = build.load_extension()
            sys.modules[EXT_NAME] = mod
            _ext = mod
        _module = extension()
        logger.info("gfx950 attention kernel loaded")
    except Exception as exc:  # noqa: BLE001 - caller keeps its stock attention
        logger.warning("gfx950 attention kernel unavailable: %s", exc)
        _module = None
    return _module
