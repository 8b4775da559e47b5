"""CPU tests of the build path of the boundary.

* The reference builds its op with ``torch.utils.cpp_extension.load(name=...,
  sources=[attn.cpp], extra_ldflags=[<kernel object>])`` (README.md:12-13,
  deploy/gfx906_attn.py:77-83, test.py:2-3). The same call, on this build's
  binding sources and its kernel library, must produce a module whose
  ``attn`` validates inputs like the product's.
* ``load_attention()``'s build-once rules (deploy/gfx906_attn.py:40-59):
  rebuild a missing or stale kernel library, record success and failure in
  marker files, and do not retry a failed build (until a source changes),
  here with a stand-in compiler in place of hipcc.
"""

import os
import sys
import textwrap
import time
from unittest import mock

import pytest
import torch

from gfx906_amd import build, loader


def test_reference_style_cpp_extension_load(tmp_path):
    from torch.utils import cpp_extension

    m = cpp_extension.load(
        name="gfx906_attn",  # test.py:2
        sources=[str(s) for s in build.BINDING_SOURCES],
        extra_ldflags=[str(build.KERNEL_LIB)],
        extra_include_paths=[str(build.INCLUDE), str(build.ROCM / "include")],
        extra_cflags=build.EXT_CFLAGS,
        build_directory=str(tmp_path))
    assert callable(m.attn) and callable(m.conv3d)
    q = torch.zeros(1, 1, 4, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="CUDA fp16"):
        m.attn(q, q, q, 0.125)


def test_product_extension_is_the_cpp_extension_build():
    # build_all() leaves torch's ninja file next to the module it produced.
    ninja = build.LIB / "build.ninja"
    assert ninja.is_file() and build.EXT_LIB.is_file()
    text = ninja.read_text()
    assert "gfx906_amd_attn_ext" in text and "-lgfx906_amd_attn" in text


FAKE_HIPCC = textwrap.dedent("""\
    #!{python}
    import os, sys
    with open(os.environ["FAKE_HIPCC_LOG"], "a") as f:
        f.write(" ".join(sys.argv[1:]) + "\\n")
    if os.environ.get("FAKE_HIPCC_FAIL"):
        sys.stderr.write("error: fake compiler failure\\n")
        sys.exit(1)
    out = sys.argv[sys.argv.index("-o") + 1]
    open(out, "wb").write(b"\\x7fELF fake")
""")


@pytest.fixture
def fake_hipcc(tmp_path, monkeypatch):
    exe = tmp_path / "hipcc"
    exe.write_text(FAKE_HIPCC.format(python=sys.executable))
    exe.chmod(0o755)
    log = tmp_path / "calls.log"
    monkeypatch.setenv("GFX906_AMD_HIPCC", str(exe))
    monkeypatch.setenv("FAKE_HIPCC_LOG", str(log))
    monkeypatch.delenv("FAKE_HIPCC_FAIL", raising=False)
    src = tmp_path / "k.hip"
    src.write_text("// kernel\n")
    lib = tmp_path / "lib" / "libk.so"

    def calls():
        return log.read_text().splitlines() if log.exists() else []

    return src, lib, calls


def _age(path, seconds):
    t = time.time() - seconds
    os.utime(path, (t, t))


def test_missing_library_is_built_once(fake_hipcc):
    src, lib, calls = fake_hipcc
    assert build.ensure_kernel_lib(lib, [src])
    assert lib.is_file() and (lib.parent / "libk.so.ok").is_file()
    (cmd,) = calls()
    assert "--offload-arch=gfx950" in cmd and str(src) in cmd
    assert build.ensure_kernel_lib(lib, [src])  # up to date: no second compile
    assert len(calls()) == 1


def test_stale_library_is_rebuilt(fake_hipcc):
    src, lib, calls = fake_hipcc
    assert build.ensure_kernel_lib(lib, [src])
    _age(lib, 100)  # the source is now newer than the library
    assert build.ensure_kernel_lib(lib, [src])
    assert len(calls()) == 2 and lib.stat().st_mtime > time.time() - 50


def test_failed_build_is_not_retried_until_a_source_changes(fake_hipcc, monkeypatch):
    src, lib, calls = fake_hipcc
    monkeypatch.setenv("FAKE_HIPCC_FAIL", "1")
    assert not build.ensure_kernel_lib(lib, [src])
    failed = lib.parent / "libk.so.failed"
    assert "fake compiler failure" in failed.read_text() and not lib.exists()
    assert not build.ensure_kernel_lib(lib, [src])  # marker: no retry
    assert len(calls()) == 1
    monkeypatch.delenv("FAKE_HIPCC_FAIL")
    _age(failed, 100)  # a source edited after the failure re-enables the build
    assert build.ensure_kernel_lib(lib, [src])
    assert len(calls()) == 2 and not failed.exists()


def test_missing_compiler_counts_as_a_failed_build(fake_hipcc, monkeypatch, tmp_path):
    src, lib, _ = fake_hipcc
    monkeypatch.setenv("GFX906_AMD_HIPCC", str(tmp_path / "no-such-hipcc"))
    assert not build.ensure_kernel_lib(lib, [src])
    assert (lib.parent / "libk.so.failed").is_file()


@pytest.fixture
def fresh_loader(monkeypatch):
    monkeypatch.setattr(loader, "_attempted", False)
    monkeypatch.setattr(loader, "_module", None)
    monkeypatch.setattr(loader, "is_gfx950", lambda: True)


def test_load_attention_returns_none_when_the_kernel_build_fails(fresh_loader):
    with mock.patch.object(build, "ensure_kernel_lib", return_value=False) as ens, \
            mock.patch.object(build, "load_extension", side_effect=AssertionError):
        assert loader.load_attention() is None
        assert loader.load_attention() is None  # cached: no second attempt
    ens.assert_called_once()


def test_load_attention_builds_a_stale_binding(fresh_loader, monkeypatch):
    mod = object()
    monkeypatch.setattr(loader, "_ext", None)
    with mock.patch.object(build, "ensure_kernel_lib", return_value=True), \
            mock.patch.object(build, "extension_stale", return_value=True), \
            mock.patch.object(build, "load_extension", return_value=mod) as load, \
            mock.patch.dict(sys.modules):
        assert loader.load_attention() is mod
    load.assert_called_once()


def test_load_attention_uses_the_built_binding(fresh_loader):
    with mock.patch.object(build, "ensure_kernel_lib", return_value=True), \
            mock.patch.object(build, "extension_stale", return_value=False), \
            mock.patch.object(build, "load_extension", side_effect=AssertionError):
        mod = loader.load_attention()
    assert mod is loader.extension() and callable(mod.attn)
