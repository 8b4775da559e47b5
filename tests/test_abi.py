"""CPU checks of the drop-in boundary: the C-ABI library loads and exports
every function include/gfx906_amd_attn.h declares, rejects bad arguments
before touching the GPU, and the torch binding loads and validates inputs.
No kernel is launched here."""

import ctypes
import os
import re
import subprocess

import pytest
import torch

import gfx906_amd
from gfx906_amd import loader

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gfx906_amd_attn.h")
HEADERS = [os.path.join(ROOT, "include", h) for h in sorted(os.listdir(os.path.join(ROOT, "include")))
           if h.endswith(".h")]


def declared_functions(headers=None):
    names = []
    for h in headers or HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names += re.findall(r"^\s*[\w\s\*]+?\b(\w+)\s*\(", text, flags=re.M)
    return names


def test_header_declares_reference_entry_points():
    names = declared_functions()
    assert "launch" in names and "attn_fwd" in names and "attn_last_error" in names
    assert {"launch_conv3d", "conv3d_fwd", "conv3d_last_error"} <= set(names)
    assert len(HEADERS) == 2


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(loader.KERNEL_LIB))
    for name in declared_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(loader.KERNEL_LIB)],
                         capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert set(declared_functions()) <= exported


def test_launch_signature_matches_reference():
    # attn.cpp:4-5: void launch(const void*, const void*, const void*, void*,
    #                           int,int,int,int,int, float, hipStream_t)
    text = re.sub(r"\s+", " ", open(HEADER).read())
    assert ("void launch(const void* q, const void* k, const void* v, void* o, int B, int H, "
            "int Sq, int Skv, int D, float scale, hipStream_t stream);") in text


@pytest.mark.parametrize("D", [0, 7, 72, 96, 100, 256, 1024])
def test_bad_head_dim_rejected_without_launch(D):
    lib = gfx906_amd.capi()
    assert lib.attn_fwd(None, None, None, None, 1, 1, 4, 4, D, 0.1, None) == 1
    assert b"head_dim" in lib.attn_last_error()
    lib.launch(None, None, None, None, 1, 1, 4, 4, D, 0.1, None)
    assert b"head_dim" in lib.attn_last_error()


def test_negative_sizes_and_null_pointers_rejected():
    lib = gfx906_amd.capi()
    assert lib.attn_fwd(None, None, None, None, -1, 1, 4, 4, 64, 0.1, None) == 1
    assert b"negative" in lib.attn_last_error()
    assert lib.attn_fwd(None, None, None, None, 1, 1, 4, 4, 64, 0.1, None) == 1
    assert b"null" in lib.attn_last_error()


def test_many_batch_heads_are_not_a_grid_limit():
    # B*H above 65535 reaches the pointer checks (no "grid too large"): the
    # grid is one-dimensional and only HIP's 2^32 work-item bound applies.
    lib = gfx906_amd.capi()
    assert lib.attn_fwd(None, None, None, None, 65536, 1, 8, 8, 8, 0.1, None) == 1
    assert b"null" in lib.attn_last_error()
    assert lib.attn_fwd(None, None, None, None, 2, 40000, 3, 5, 64, 0.1, None) == 1
    assert b"null" in lib.attn_last_error()
    # 2^23 query tiles of 512 threads reach 2^32 work items.
    assert lib.attn_fwd(None, None, None, None, 1 << 14, 1 << 9, 256, 8, 64, 0.1, None) == 1
    assert b"grid too large" in lib.attn_last_error()


def test_empty_problem_is_a_no_op():
    lib = gfx906_amd.capi()
    assert lib.attn_fwd(None, None, None, None, 0, 4, 4, 4, 64, 0.1, None) == 0
    assert lib.attn_last_error() is None


def test_torch_extension_loads_and_validates_on_cpu():
    ext = gfx906_amd.extension()
    q = torch.zeros(1, 1, 4, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="CUDA fp16"):
        ext.attn(q, q, q, 0.1)


def test_load_attention_returns_none_without_gfx950():
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    loader._attempted = False
    assert gfx906_amd.load_attention() is None
    assert not gfx906_amd.is_gfx950()


def test_product_package_never_imports_oracle():
    pkg = os.path.join(ROOT, "gfx906_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in re.sub(r"#.*|//.*", "", text), f


def test_flops_formula():
    # flops_probe.py:18: 4*B*H*S*S*D
    assert gfx906_amd.flops(1, 16, 16384, 16384, 128) == 2_199_023_255_552


# -- attn_fwd_ex: rejected before any HIP call ---------------------------------------------

P = ctypes.c_void_p(0x10000)  # aligned, never dereferenced: every case below is rejected


def _ex(B=1, H=2, Sq=16, Skv=16, D=64, dtype=0, q=None, k=None, v=None, o=None, ptrs=None):
    lib = gfx906_amd.capi()
    # 3-tuples are {batch, head, seq} with a contiguous head dim
    arr = [None if s is None else (ctypes.c_longlong * 4)(*s, *((1,) if len(s) == 3 else ()))
           for s in (q, k, v, o)]
    pq, pk, pv, po = ptrs or (P, P, P, P)
    rc = lib.attn_fwd_ex(pq, pk, pv, po, B, H, Sq, Skv, D, 0.1, None, dtype, *arr)
    return rc, lib.attn_last_error()


def test_ex_rejects_unknown_dtype():
    assert _ex(dtype=2) == (1, b"attn: dtype must be ATTN_DTYPE_F16 or ATTN_DTYPE_BF16")


@pytest.mark.parametrize("which", ["q", "k", "v"])
def test_ex_rejects_input_strides_not_multiple_of_8(which):
    rc, err = _ex(**{which: (2 * 16 * 64, 16 * 64, 60)})
    assert rc == 1 and b"multiples of 8" in err
    rc, err = _ex(**{which: (-8, 16 * 64, 64)})
    assert rc == 1 and b"non-negative" in err


def test_ex_rejects_output_strides_and_overlap():
    assert _ex(o=(2 * 16 * 64, 16 * 64, 62))[1].startswith(b"attn: o strides must")
    # all query rows of a head written to one row
    assert b"overlap" in _ex(o=(2 * 64, 64, 0))[1]
    # heads interleaved onto each other: head stride smaller than a row
    assert b"overlap" in _ex(o=(2 * 16 * 64, 32, 64 * 2))[1]


def test_ex_rejects_misaligned_pointers():
    rc, err = _ex(ptrs=(ctypes.c_void_p(0x10008), P, P, P))
    assert rc == 1 and b"aligned" in err
    rc, err = _ex(ptrs=(P, P, P, ctypes.c_void_p(0x10004)))
    assert rc == 1 and b"aligned" in err


def test_ex_rejects_huge_kv_sequence_stride():
    rc, err = _ex(k=(0, 0, (1 << 24) + 8))
    assert rc == 1 and b"2^24" in err


def test_ex_null_strides_mean_contiguous_and_empty_is_no_op():
    lib = gfx906_amd.capi()
    assert lib.attn_fwd_ex(None, None, None, None, 0, 2, 16, 16, 64, 0.1, None, 1,
                           None, None, None, None) == 0
    assert lib.attn_last_error() is None


def test_header_dtype_codes():
    text = open(HEADER).read()
    assert re.search(r"#define ATTN_DTYPE_F16 0\b", text)
    assert re.search(r"#define ATTN_DTYPE_BF16 1\b", text)


def test_launch_conv3d_signature_matches_reference():
    # hip_conv/conv3d_kernel.hip:218-225 (stream: hipStream_t, void* in the binding's copy)
    text = re.sub(r"\s+", " ", open(os.path.join(ROOT, "include", "gfx906_amd_conv3d.h")).read())
    assert ("void launch_conv3d(const void* x, const void* w, const void* bias, const void* res, "
            "void* out, int nB, int D, int H, int W, int C, int K, int T, int R, int S, int sd, "
            "int sh, int sw, int Z, int P, int Q, long M, long xsn, long xsd, long xsh, long xsw, "
            "long osn, long osz, long osp, long osq, long rsn, long rsz, long rsp, long rsq, "
            "hipStream_t stream);") in text


def _conv(**kw):
    """conv3d_fwd with a valid 1x8x4x6x6 -> 8x3x3x3 problem, fields overridden by kw."""
    lib = ctypes.CDLL(str(loader.KERNEL_LIB))
    lib.conv3d_fwd.restype = ctypes.c_int
    lib.conv3d_last_error.restype = ctypes.c_char_p
    v = dict(x=0x10000, w=0x20000, bias=0, res=0, out=0x30000, nB=1, D=4, H=6, W=6, C=8, K=8,
             T=3, R=3, S=3, sd=1, sh=1, sw=1, Z=2, P=4, Q=4, M=32,
             xs=(4 * 6 * 6 * 8, 6 * 6 * 8, 6 * 8, 8), os=(2 * 4 * 4 * 8, 4 * 4 * 8, 4 * 8, 8),
             rs=(0, 0, 0, 0))
    v.update(kw)
    args = ([ctypes.c_void_p(v[k]) for k in ("x", "w", "bias", "res", "out")]
            + [ctypes.c_int(v[k]) for k in ("nB", "D", "H", "W", "C", "K", "T", "R", "S", "sd",
                                             "sh", "sw", "Z", "P", "Q")]
            + [ctypes.c_long(v["M"])] + [ctypes.c_long(s) for s in (*v["xs"], *v["os"], *v["rs"])]
            + [ctypes.c_void_p(0)])
    return lib.conv3d_fwd(*args), lib.conv3d_last_error()


@pytest.mark.parametrize("kw,msg", [
    (dict(C=12), b"multiples of 8"),
    (dict(K=4), b"multiples of 8"),
    (dict(Z=3), b"VALID"),
    (dict(M=31), b"nB*Z*P*Q"),
    (dict(sd=0), b"strides must be positive"),
    (dict(T=5, D=4), b"VALID"),
    (dict(x=0x10008), b"aligned"),
    (dict(bias=0x10004), b"aligned"),
    (dict(xs=(4 * 6 * 6 * 8, 6 * 6 * 8, 6 * 8, 12)), b"multiples of 8"),
    (dict(x=0), b"null"),
    (dict(xs=(1 << 30, 6 * 6 * 8, 6 * 8, 8), nB=2, M=64), b"2^31"),
])
def test_conv3d_rejects_without_launch(kw, msg):
    rc, err = _conv(**kw)
    assert rc == 1 and msg in err, err


def test_ex_head_dim_stride_rules():
    # outside D == 512 with token-contiguous k/v the head dim must be contiguous
    rc, err = _ex(D=64, q=(2 * 16 * 64, 16 * 64, 1, 16))
    assert rc == 1 and b"head dim must be contiguous" in err
    rc, err = _ex(D=512, Skv=64, k=(2 * 64 * 512, 64 * 512, 512, 2))  # k d-strided, not token-contig
    assert rc == 1 and b"head dim must be contiguous" in err
    # token-contiguous k/v: Skv % 8, stride multiples, span
    tk = (2 * 512 * 64, 512 * 64, 1, 64)
    rc, err = _ex(D=512, Skv=63, k=(2 * 512 * 64, 512 * 64, 1, 64), v=(2 * 512 * 64, 512 * 64, 1, 64))
    assert rc == 1 and b"Skv % 8" in err
    rc, err = _ex(D=512, Skv=64, k=(2 * 512 * 64, 512 * 64, 1, 68), v=tk)
    assert rc == 1 and b"multiples of 8" in err
    rc, err = _ex(D=512, Skv=64, k=(0, 0, 1, 1 << 22), v=(0, 0, 1, 1 << 22))
    assert rc == 1 and b"2^30" in err
    rc, err = _ex(D=512, Skv=64, k=tk, v=tk, ptrs=(P, ctypes.c_void_p(0x10008), P, P))
    assert rc == 1 and b"16-byte" in err
    # ... with q and o of any strides, but o elements must not overlap
    rc, err = _ex(D=512, Skv=64, k=tk, v=tk, o=(2 * 16 * 512, 16 * 512, 512, 0))
    assert rc == 1 and b"overlap" in err


# -- attn_fwd_split: workspace sizing and rejections (no GPU: plans assume 256 CUs) ------

def test_split_workspace_bytes():
    lib = gfx906_amd.capi()
    assert lib.attn_split_workspace_bytes(1, 16, 16384, 16384, 128) == 0   # fills the GPU
    assert lib.attn_split_workspace_bytes(1, 4, 8192, 8192, 512) == 0      # c4: 256 workgroups
    # VAE 64x64: 32 query tiles of 128 rows; 8 splits of 512 keys
    assert lib.attn_split_workspace_bytes(1, 1, 4096, 4096, 512) == 8 * 4096 * (512 + 2) * 4 + 16
    # too few key tiles to split (fewer than 8 = 2 splits x 4 tiles)
    assert lib.attn_split_workspace_bytes(1, 1, 300, 400, 128) == 0
    # 72 query tiles: 3 splits fill the 256 CUs in one round (4 would take two)
    assert lib.attn_split_workspace_bytes(1, 1, 9216, 9216, 512) == 3 * 9216 * (512 + 2) * 4 + 16
    # 200 query tiles: a split would take two rounds of half the work, so none
    assert lib.attn_split_workspace_bytes(1, 1, 25600, 4096, 512) == 0
    # D = 128, 64 key tiles: 16 splits of 4 tiles; 11 or 13 would leave 6 or 5
    # tiles per split, which the kernel's groups of four tiles run as 8
    assert lib.attn_split_workspace_bytes(1, 1, 4096, 4096, 128) == 16 * 4096 * (128 + 2) * 4 + 16
    # D = 64 runs two workgroups per CU: 4 splits (256 workgroups, one per CU)
    # beat 8 (512, two per CU) on 8 heads of 2048 queries
    assert lib.attn_split_workspace_bytes(1, 8, 2048, 2048, 64) == 4 * 8 * 2048 * (64 + 2) * 4 + 16
    for bad in ((0, 1, 8, 8, 64), (1, 1, 8, 0, 64), (1, 1, 8, 8, 96)):
        assert lib.attn_split_workspace_bytes(*bad) == 0


@pytest.mark.parametrize("n,D,H,Skv,want", [
    (5, 128, 1, 4096, 5),      # 64 tiles: 13 per range, the last 12
    (7, 128, 1, 4096, 7),      # 10 per range, the last 4
    (12, 128, 1, 4096, 11),    # 6 per range (5 would make 13 ranges): 11 ranges, the last 4
    (13, 128, 1, 4096, 13),    # 5 per range, the last 4
    (64, 128, 1, 4096, 64),    # one tile per range
    (99, 128, 1, 4096, 64),    # at most one range per tile
    (3, 512, 1, 1000, 3),      # 32 tiles of 32 keys: 11, 11, 10
    (1, 512, 1, 4096, 1),      # no split
    (2, 128, 16, 16384, 2),    # also a grid that fills the GPU
])
def test_split_count_forced_by_environment(monkeypatch, n, D, H, Skv, want):
    """GFX906_AMD_ATTN_NSPLIT (tests) replaces the estimate's count: ranges of
    ceil(tiles / n) whole tiles, as many as that takes."""
    lib = gfx906_amd.capi()
    monkeypatch.setenv("GFX906_AMD_ATTN_NSPLIT", str(n))
    got = lib.attn_split_workspace_bytes(1, H, 1024, Skv, D)
    assert got == (0 if want == 1 else want * H * 1024 * (D + 2) * 4 + 16)
    monkeypatch.delenv("GFX906_AMD_ATTN_NSPLIT")
    assert lib.attn_split_workspace_bytes(1, 16, 16384, 16384, 128) == 0


def test_split_static_scratch_capacity_and_validation():
    lib = gfx906_amd.capi()
    cap = lib.attn_split_scratch_capacity()
    assert cap == 96 << 20
    # One D=512 head of 24576 queries over 65536 keys splits in four with a
    # caller workspace (three rounds of 192 workgroups): 4*24576*(512+2)*4
    # bytes, more than the static scratch holds. attn_fwd_split_static then
    # takes the best plan that fits (here none: two splits need 101 MB); the
    # GPU test checks that it runs and equals the unsplit call.
    need = lib.attn_split_workspace_bytes(1, 1, 24576, 65536, 512)
    assert need == 4 * 24576 * (512 + 2) * 4 + 16 > cap
    assert 2 * 24576 * (512 + 2) * 4 + 16 > cap
    # Arguments are validated as for attn_fwd_split, before any HIP call.
    assert lib.attn_split_workspace_bytes(1, 1, 4096, 4096, 512) <= cap
    rc = lib.attn_fwd_split_static(None, None, None, None, 1, 1, 4096, 4096, 512, 0.1, None, 0,
                                   None, None, None, None)
    assert rc == 1 and b"null" in lib.attn_last_error()


def test_split_rejects_missing_or_short_workspace():
    lib = gfx906_amd.capi()
    need = lib.attn_split_workspace_bytes(1, 1, 4096, 4096, 512)
    for ws, nbytes in ((None, need), (P, need - 16), (ctypes.c_void_p(0x10008), need)):
        rc = lib.attn_fwd_split(P, P, P, P, 1, 1, 4096, 4096, 512, 0.04, None, 0,
                                None, None, None, None, ws, nbytes)
        assert rc == 1 and b"workspace" in lib.attn_last_error()


def test_c_harness_links_the_library_and_checks_usage(tmp_path):
    # The torch-free caller of launch() (gfx906_amd/csrc/launch_harness.cpp)
    # is built with the library and resolves it from its own directory; bad
    # usage and missing inputs fail before any HIP call.
    from gfx906_amd.build import HARNESS

    assert HARNESS.is_file()
    deps = subprocess.run(["ldd", str(HARNESS)], capture_output=True, text=True).stdout
    assert str(loader.KERNEL_LIB) in deps
    assert subprocess.run([str(HARNESS)], capture_output=True).returncode == 1
    res = subprocess.run([str(HARNESS), str(tmp_path), "1", "1", "4", "4", "64", "0.1", "1"],
                         capture_output=True, text=True)
    assert res.returncode == 1 and "cannot read" in res.stderr
