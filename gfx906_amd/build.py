"""In-tree build of the gfx950 attention libraries.

Two shared objects and one program are produced under ``gfx906_amd/lib/``:

* ``libgfx906_amd_attn.so`` -- the HIP kernels and the C ABIs declared in
  ``include/gfx906_amd_attn.h`` and ``include/gfx906_amd_conv3d.h``, compiled
  by ``hipcc --offload-arch=gfx950``. It plays the part of the reference's
  separately compiled kernel objects (``attn_kernel.gfx906.o``,
  ``conv3d_kernel.<arch>.o``; README.md:12, deploy/gfx906_attn.py:40-59).
* ``gfx906_amd_attn_ext.so`` -- the PyTorch binding (``attn(q, k, v, scale)``
  and ``conv3d(...)``), built the way the reference builds its own
  (README.md:13, deploy/gfx906_attn.py:77-83): ``torch.utils.cpp_extension
  .load`` over the plain C++ binding sources with the kernel library in
  ``extra_ldflags``. The build directory is ``gfx906_amd/lib`` itself, so the
  module sits next to the kernel library and finds it through an ``$ORIGIN``
  run path.
* ``launch_harness`` -- a torch-free C++ program that calls ``launch()``
  through the C ABI on device buffers it allocates itself, as the
  reference's ``micro3.hip`` does (micro3.hip:4-17).

:func:`build_all` rebuilds both every time it is called. :func:`ensure_kernel_lib`
is the build-once path the loader uses: rebuild a missing or stale library,
record the outcome in a marker file, and do not retry a failed build until
one of its sources changes.
"""

from __future__ import annotations

import logging
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
LIB = PKG / "lib"
KERNEL_LIB = LIB / "libgfx906_amd_attn.so"
EXT_NAME = "gfx906_amd_attn_ext"
EXT_LIB = LIB / f"{EXT_NAME}.so"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

logger = logging.getLogger("gfx906_amd")

ARCH = "gfx950"
# Packed fp32 VALU ops are disabled: hipcc must not form v_pk_{add,mul,fma}_f32.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
    # MFMAs the compiler emits keep their accumulators in VGPRs. Only
    # attn_fwd_d512w (one wave per SIMD, 512 registers) is affected: its
    # score MFMAs then accumulate in VGPRs beside Q, while its O^T
    # accumulator is pinned to AGPRs by inline asm. Every other kernel has at
    # most 256 registers per lane and is compiled identically either way.
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
]

KERNEL_SOURCES = [CSRC / "attn_kernel.hip", CSRC / "conv3d_kernel.hip"]
# A torch-free C caller of launch() (the reference's micro3.hip pattern),
# linked against the kernel library.
HARNESS_SOURCE = CSRC / "launch_harness.cpp"
HARNESS = LIB / "launch_harness"
BINDING_SOURCES = [CSRC / "attn.cpp", CSRC / "conv3d.cpp", CSRC / "module.cpp"]
# The binding is host C++ only; HIP types come from the runtime headers.
EXT_CFLAGS = ["-O2", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1"]
EXT_LDFLAGS = [f"-L{LIB}", "-lgfx906_amd_attn", "-lc10_hip", "-ltorch_hip",
               f"-L{ROCM / 'lib'}", "-lamdhip64", "-Wl,-rpath,'$$ORIGIN'"]


def hipcc() -> str:
    """The HIP compiler: $GFX906_AMD_HIPCC, else hipcc on PATH, else ROCm's."""
    return (os.environ.get("GFX906_AMD_HIPCC") or shutil.which("hipcc")
            or str(ROCM / "bin" / "hipcc"))


def _kernel_lib_command(sources, out) -> list:
    return [hipcc(), *HIP_FLAGS, "-shared", f"-I{INCLUDE}", *map(str, sources), "-o", str(out)]


def _run(cmd, cwd=None):
    res = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(map(str, cmd))}\n{res.stdout}\n{res.stderr}")
    return res


def build_kernel_lib(extra_flags=()) -> Path:
    """Compile the HIP sources into the C-ABI shared library."""
    LIB.mkdir(exist_ok=True)
    tmp = KERNEL_LIB.with_suffix(".so.tmp")
    _run([*_kernel_lib_command(KERNEL_SOURCES, tmp), *extra_flags])
    os.replace(tmp, KERNEL_LIB)
    return KERNEL_LIB


def load_extension(verbose=False):
    """torch.utils.cpp_extension.load of the binding into gfx906_amd/lib
    (ninja rebuilds what is out of date); returns the module."""
    from torch.utils import cpp_extension

    LIB.mkdir(exist_ok=True)
    return cpp_extension.load(
        name=EXT_NAME,
        sources=[str(s) for s in BINDING_SOURCES],
        extra_cflags=EXT_CFLAGS,
        extra_include_paths=[str(INCLUDE), str(ROCM / "include")],
        extra_ldflags=EXT_LDFLAGS,
        build_directory=str(LIB),
        verbose=verbose)


def build_extension() -> Path:
    """Compile the binding from scratch (its objects and module are removed
    first, so the sources really are compiled)."""
    for f in [EXT_LIB, *(LIB / (s.stem + ".o") for s in BINDING_SOURCES)]:
        f.unlink(missing_ok=True)
    load_extension()
    return EXT_LIB


def build_harness() -> Path:
    """Compile the C caller of launch() against the kernel library (host code
    only; the library is found through an $ORIGIN run path)."""
    LIB.mkdir(exist_ok=True)
    tmp = HARNESS.with_suffix(".tmp")
    _run([hipcc(), "-O2", "-std=c++17", f"-I{INCLUDE}", str(HARNESS_SOURCE), "-o", str(tmp),
          f"-L{LIB}", "-lgfx906_amd_attn", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, HARNESS)
    return HARNESS


def build_all() -> None:
    build_kernel_lib()
    build_extension()
    build_harness()


# -- build once, for the loader -----------------------------------------------------------

def _newest_mtime(paths) -> float:
    return max(p.stat().st_mtime for p in paths if p.exists())


def kernel_lib_inputs() -> list:
    return [*KERNEL_SOURCES, *sorted(INCLUDE.glob("*.h"))]


def ensure_kernel_lib(lib: Path = KERNEL_LIB, sources=None) -> bool:
    """Make sure `lib` exists and is not older than its sources.

    A missing or stale library is rebuilt with :func:`hipcc`. Success writes
    ``<lib>.ok`` (the command and the compiler's messages) and removes any
    ``<lib>.failed``; failure writes ``<lib>.failed`` (the end of the
    compiler's output) and returns False. While ``<lib>.failed`` is newer
    than every source, no rebuild is tried again (the reference's
    ``.build_failed`` rule, deploy/gfx906_attn.py:40-59, except that editing
    a source re-enables the build).
    """
    sources = [Path(s) for s in (sources if sources is not None else kernel_lib_inputs())]
    lib = Path(lib)
    ok, failed = lib.with_name(lib.name + ".ok"), lib.with_name(lib.name + ".failed")
    newest = _newest_mtime(sources)
    if lib.is_file() and lib.stat().st_mtime >= newest:
        return True
    if failed.is_file() and failed.stat().st_mtime >= newest:
        return False
    lib.parent.mkdir(parents=True, exist_ok=True)
    tmp = lib.with_name(lib.name + ".tmp")
    cmd = _kernel_lib_command([s for s in sources if s.suffix == ".hip"], tmp)
    try:
        res = subprocess.run(cmd, capture_output=True, text=True)
        built = res.returncode == 0 and tmp.is_file()
        log = res.stdout + res.stderr
    except OSError as exc:  # compiler missing
        built, log = False, str(exc)
    if built:
        os.replace(tmp, lib)
        ok.write_text(" ".join(cmd) + "\n" + log)
        failed.unlink(missing_ok=True)
        return True
    tmp.unlink(missing_ok=True)
    failed.write_text(log[-4000:])
    logger.warning("gfx950 kernel library build failed: %s", log[-500:])
    return False


def extension_stale() -> bool:
    """Whether the binding module is missing or older than its sources or
    the kernel library's header."""
    if not EXT_LIB.is_file():
        return True
    inputs = [*BINDING_SOURCES, CSRC / "bindings.h", *INCLUDE.glob("*.h")]
    return EXT_LIB.stat().st_mtime < _newest_mtime(inputs)


if __name__ == "__main__":
    build_all()
    print(KERNEL_LIB, EXT_LIB, file=sys.stderr)
