"""In-tree build of the gfx950 attention libraries.

Two shared objects are produced under ``gfx906_amd/lib/``:

* ``libgfx906_amd_attn.so`` -- the HIP kernels and the C ABIs declared in
  ``include/gfx906_amd_attn.h`` and ``include/gfx906_amd_conv3d.h``, compiled
  by ``hipcc --offload-arch=gfx950``. This plays the part of the reference's
  separately compiled ``attn_kernel.o`` and ``conv3d_kernel.<arch>.o``
  (README.md:12, deploy/gfx906_attn.py:40-59, gfx906_kitchen.py:58-76).
* ``gfx906_amd_attn_ext.so`` -- the PyTorch bindings ``attn(q, k, v, scale)``
  and ``conv3d(x, w, bias, res, out, dims, xs, os, rs)`` (counterparts of
  the reference's attn.cpp and hip_conv/conv3d.cpp built by
  ``cpp_extension.load``, README.md:13), linked against the library above
  with an ``$ORIGIN`` rpath so the pair loads from the package directory.

Both are rebuilt on every call of :func:`build_all`; nothing here runs at
import time of the package.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "lib"
KERNEL_LIB = LIB / "libgfx906_amd_attn.so"
CEILING_LIB = LIB / "libgfx906_amd_ceiling.so"
EXT_NAME = "gfx906_amd_attn_ext"
EXT_LIB = LIB / f"{EXT_NAME}.so"

ARCH = "gfx950"
# Packed fp32 VALU ops are disabled: hipcc must not form v_pk_{add,mul,fma}_f32.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
]


def hipcc() -> str:
    return shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def _run(cmd, cwd=None):
    res = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(map(str, cmd))}\n{res.stdout}\n{res.stderr}")
    return res


KERNEL_SOURCES = ["attn_kernel.hip", "conv3d_kernel.hip"]
BINDING_SOURCES = ["attn.cpp", "conv3d.cpp", "module.cpp"]


def build_kernel_lib(extra_flags=()) -> Path:
    """Compile the HIP sources into the C-ABI shared library."""
    LIB.mkdir(exist_ok=True)
    tmp = KERNEL_LIB.with_suffix(".so.tmp")
    _run([hipcc(), *HIP_FLAGS, *extra_flags, "-shared", f"-I{ROOT / 'include'}",
          *[str(CSRC / f) for f in KERNEL_SOURCES], "-o", str(tmp)])
    os.replace(tmp, KERNEL_LIB)
    return KERNEL_LIB


def build_ceiling_lib() -> Path:
    """Compile the MFMA throughput probe (bench.py --ceiling) into its own library."""
    LIB.mkdir(exist_ok=True)
    tmp = CEILING_LIB.with_suffix(".so.tmp")
    _run([hipcc(), *HIP_FLAGS, "-shared", str(CSRC / "mfma_ceiling.hip"), "-o", str(tmp)])
    os.replace(tmp, CEILING_LIB)
    return CEILING_LIB


def build_extension() -> Path:
    """Compile the binding sources into the torch extension, linked to the kernel lib.

    The binding is plain C++ (no device code), so it is compiled by the host
    compiler with torch's include and library paths; no source translation
    step is involved.
    """
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    LIB.mkdir(exist_ok=True)
    incs = [*cpp_extension.include_paths(device_type="cuda"), str(ROOT / "include"),
            sysconfig.get_paths()["include"]]
    libdirs = cpp_extension.library_paths(device_type="cuda")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cxx = shutil.which("g++") or "c++"
    tmp = EXT_LIB.with_suffix(".so.tmp")
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-w",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           *[f"-I{i}" for i in incs],
           *[str(CSRC / f) for f in BINDING_SOURCES], "-o", str(tmp),
           f"-L{LIB}", "-lgfx906_amd_attn",
           *[f"-L{d}" for d in libdirs],
           "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch_hip", "-ltorch", "-ltorch_python",
           "-lamdhip64", "-Wl,-rpath,$ORIGIN"]
    _run(cmd)
    os.replace(tmp, EXT_LIB)
    return EXT_LIB


def build_all() -> None:
    build_kernel_lib()
    build_ceiling_lib()
    build_extension()


if __name__ == "__main__":
    build_all()
    print(KERNEL_LIB, EXT_LIB, file=sys.stderr)
