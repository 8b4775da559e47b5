"""attn_fwd_split_static (split key ranges, workspace in the library's static
device scratch) through the C ABI:

* against attn_fwd_split with a caller workspace, on two calls in a row (the
  second smaller, so it runs on what the first left in the scratch): both run
  the same split plan and kernels, so the outputs must be bit-identical; both
  are also held to the north-star bar against the CPU oracle;
* a problem whose caller-workspace plan does not fit the scratch runs with
  the best plan that does (here none) and equals attn_fwd_ex bit for bit;
* captured in a CUDA graph and replayed, with eager calls between replays;
* issued on three streams at once, overlapping: the calls that use the
  scratch are ordered on the GPU, so every result equals its serial one;
* launch() and attn_fwd(), which split small grids through the same scratch.
"""

import ctypes

import pytest
import torch

import gfx906_amd
from oracle.attention import MAX_ABS_TOL, MEAN_ABS_TOL, error_stats, make_inputs, sdpa_math_fp32

pytestmark = pytest.mark.gpu


def _split(lib, q, k, v, scale, o=None):
    B, H, Sq, D = q.shape
    Skv = k.shape[2]
    need = lib.attn_split_workspace_bytes(B, H, Sq, Skv, D)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    o = torch.empty_like(q) if o is None else o
    rc = lib.attn_fwd_split(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H, Sq,
                            Skv, D, scale, torch.cuda.current_stream().cuda_stream, 0,
                            None, None, None, None, ctypes.c_void_p(ws.data_ptr()), need)
    assert rc == 0, lib.attn_last_error()
    return o, need


def _static(lib, q, k, v, scale, o=None):
    B, H, Sq, D = q.shape
    o = torch.full_like(q, float("nan")) if o is None else o
    rc = lib.attn_fwd_split_static(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H,
                                   Sq, k.shape[2], D, scale,
                                   torch.cuda.current_stream().cuda_stream, 0,
                                   None, None, None, None)
    assert rc == 0, lib.attn_last_error()
    return o


def _ex(lib, q, k, v, scale):
    B, H, Sq, D = q.shape
    o = torch.full_like(q, float("nan"))
    rc = lib.attn_fwd_ex(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H, Sq,
                         k.shape[2], D, scale, torch.cuda.current_stream().cuda_stream, 0,
                         None, None, None, None)
    assert rc == 0, lib.attn_last_error()
    return o


def _launch(lib, q, k, v, scale, o):
    B, H, Sq, D = q.shape
    lib.launch(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H, Sq, k.shape[2], D,
               float(scale), torch.cuda.current_stream().cuda_stream)
    assert lib.attn_last_error() is None
    return o


def _inputs(B, H, Sq, Skv, D, seed):
    qc, kc, vc = make_inputs(B, H, Sq, Skv, D, seed=seed)
    return (qc, kc, vc), (qc.cuda(), kc.cuda(), vc.cuda())


def _check_rows(out, qc, kc, vc, scale, what):
    Sq = qc.shape[2]
    rows = torch.arange(0, Sq, max(1, Sq // 128))
    ref = sdpa_math_fp32(qc[:, :, rows], kc, vc, scale)
    mx, mn = error_stats(out[:, :, rows].float().cpu(), ref)
    print(f"  {what} vs oracle: max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)
    assert mx <= MAX_ABS_TOL and mn <= MEAN_ABS_TOL


@pytest.mark.parametrize("first,second", [
    ((1, 1, 4096, 4096, 512), (1, 1, 1000, 1500, 512)),  # one VAE head, then a smaller one
    ((1, 4, 2048, 3000, 128), (1, 2, 700, 900, 128)),
    ((2, 2, 1024, 2048, 64), (1, 1, 300, 1111, 40)),
])
def test_static_scratch_matches_caller_workspace(first, second):
    lib = gfx906_amd.capi()
    for n, (B, H, Sq, Skv, D) in enumerate((first, second)):
        print(f"case: call {n + 1} B{B} H{H} Sq{Sq} Skv{Skv} D{D}", flush=True)
        (qc, kc, vc), (q, k, v) = _inputs(B, H, Sq, Skv, D, 1000 * n + D + Sq)
        scale = D ** -0.5
        a, need = _split(lib, q, k, v, scale)
        assert 0 < need <= lib.attn_split_scratch_capacity()  # the call really splits
        b = _static(lib, q, k, v, scale)
        torch.cuda.synchronize()
        assert torch.equal(a, b)
        _check_rows(b, qc, kc, vc, scale, "static")
    # D = 64 runs two workgroups per CU: 4 splits (256 workgroups, one per CU)
    # beat 8 (512, two per CU) on 8 heads of 2048 queries
    assert lib.attn_split_workspace_bytes(1, 8, 2048, 2048, 64) == 4 * 8 * 2048 * (64 + 2) * 4 + 16
    for bad in ((0, 1, 8, 8, 64), (1, 1, 8, 0, 64), (1, 1, 8, 8, 96)):
        assert lib.attn_split_workspace_bytes(*bad) == 0


def test_static_scratch_plan_capped_by_capacity():
    # A caller workspace would take four splits (201 MB); two do not fit the
    # 96 MiB scratch either, so the static call runs unsplit.
    lib = gfx906_amd.capi()
    B, H, Sq, Skv, D = 1, 1, 24576, 65536, 512
    print(f"case: capped plan B{B} H{H} Sq{Sq} Skv{Skv} D{D}", flush=True)
    assert lib.attn_split_workspace_bytes(B, H, Sq, Skv, D) > lib.attn_split_scratch_capacity()
    (qc, kc, vc), (q, k, v) = _inputs(B, H, Sq, Skv, D, 77)
    scale = D ** -0.5
    a = _ex(lib, q, k, v, scale)
    b = _static(lib, q, k, v, scale)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    _check_rows(b, qc, kc, vc, scale, "capped static")


def test_static_scratch_under_graph_capture():
    lib = gfx906_amd.capi()
    B, H, Sq, Skv, D = 1, 1, 4096, 4096, 512
    print(f"case: graph capture B{B} H{H} Sq{Sq} Skv{Skv} D{D}", flush=True)
    (qc, kc, vc), (q, k, v) = _inputs(B, H, Sq, Skv, D, 91)
    (_, _, _), (q2, k2, v2) = _inputs(1, 2, 1500, 3000, 128, 92)
    scale = D ** -0.5
    ref, need = _split(lib, q, k, v, scale)
    ref2, need2 = _split(lib, q2, k2, v2, 128 ** -0.5)
    assert 0 < need <= lib.attn_split_scratch_capacity() and need2 > 0
    o = torch.full_like(q, float("nan"))
    _static(lib, q, k, v, scale, o)  # outside capture: sets the device's scratch up
    torch.cuda.synchronize()
    assert torch.equal(o, ref)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _static(lib, q, k, v, scale, o)
    for r in range(3):
        o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        print(f"  replay {r}", flush=True)
        assert torch.equal(o, ref)
        # eager work between replays, through the same scratch
        e = _static(lib, q2, k2, v2, 128 ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(e, ref2)
    _check_rows(o, qc, kc, vc, scale, "replayed static")


def test_static_scratch_ordered_across_streams():
    lib = gfx906_amd.capi()
    cases = [(1, 1, 4096, 16384, 512), (1, 1, 2048, 4096, 512), (1, 2, 1024, 6000, 128),
             (1, 1, 1024, 1024, 64)]
    data, refs = [], []
    for n, (B, H, Sq, Skv, D) in enumerate(cases):
        (_, _, _), (q, k, v) = _inputs(B, H, Sq, Skv, D, 300 + n)
        ref, need = _split(lib, q, k, v, D ** -0.5)
        assert 0 < need <= lib.attn_split_scratch_capacity()
        data.append((q, k, v, D ** -0.5))
        refs.append(ref)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream(), torch.cuda.Stream()]
    main = torch.cuda.current_stream()
    for it in range(8):
        print(f"case: three streams, iteration {it}", flush=True)
        outs = [[torch.full_like(d[0], float("nan")) for d in data] for _ in streams]
        for s in streams:
            s.wait_stream(main)
        # Each case runs on every stream, the streams interleaved call by call:
        # the static entry point on some, launch() on the others.
        for n, (q, k, v, scale) in enumerate(data):
            for j, s in enumerate(streams):
                with torch.cuda.stream(s):
                    if (n + j + it) % 2:
                        _static(lib, q, k, v, scale, outs[j][n])
                    else:
                        _launch(lib, q, k, v, scale, outs[j][n])
        torch.cuda.synchronize()
        for j in range(len(streams)):
            for n in range(len(data)):
                assert torch.equal(outs[j][n], refs[n]), (it, j, n)


def test_launch_and_attn_fwd_split_small_grids():
    # One VAE head (32 query tiles on 256 CUs): launch() and attn_fwd() split
    # the keys in the static scratch, with attn_fwd_split's plan.
    lib = gfx906_amd.capi()
    B, H, Sq, Skv, D = 1, 1, 4096, 4096, 512
    print(f"case: launch split B{B} H{H} Sq{Sq} Skv{Skv} D{D}", flush=True)
    (qc, kc, vc), (q, k, v) = _inputs(B, H, Sq, Skv, D, 55)
    scale = D ** -0.5
    ref, need = _split(lib, q, k, v, scale)
    assert need > 0
    a = _launch(lib, q, k, v, scale, torch.full_like(q, float("nan")))
    b = torch.full_like(q, float("nan"))
    assert lib.attn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), b.data_ptr(), B, H, Sq, Skv, D,
                        scale, torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(a, ref) and torch.equal(b, ref)
    _check_rows(a, qc, kc, vc, scale, "launch")
