"""The op's kernels under HIP graph capture (torch.cuda.CUDAGraph): captured
once after an eager warm-up, replayed several times with the program's own
eager work and synchronisations in between, every replay compared bit for bit
with the eager result. Covers the attention path without and with split key
ranges (a workspace from the graph's pool and the combine kernel), the
token-contiguous D = 512 path, and conv3d."""

import pytest
import torch

import gfx906_amd
from gfx906_amd import kitchen
from oracle.attention import make_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda"
CL = torch.channels_last_3d


def replay_and_check(fn, out, expect, replays=3):
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    for i in range(replays):
        out.zero_()
        junk = torch.randn(1 << 20, device=DEV) * 3  # eager work between replays
        junk.sum().item()
        g.replay()
        torch.cuda.synchronize()
        print(f"replay {i}: equal {torch.equal(out, expect)}", flush=True)
        assert torch.equal(out, expect), f"replay {i} differs"


@pytest.mark.parametrize("B,H,Sq,Skv,D", [(1, 8, 1024, 1024, 128),   # whole grid
                                          (1, 1, 200, 3000, 64),     # split key ranges
                                          (2, 3, 77, 129, 40),       # padded head dim
                                          (2, 16, 4096, 77, 64),     # K/V-resident kernel
                                          (1, 8, 4096, 256, 512),    # D = 512, 32 rows/wave
                                          (1, 2, 300, 700, 512)])    # D = 512, split
def test_attention_graph_replays(B, H, Sq, Skv, D):
    q, k, v = (t.to(DEV) for t in make_inputs(B, H, Sq, Skv, D, 1.0, 1.0, seed=Sq + Skv))
    expect = gfx906_amd.attn(q, k, v, D ** -0.5)
    torch.cuda.synchronize()
    out = torch.empty_like(expect)
    replay_and_check(lambda: gfx906_amd.attn(q, k, v, D ** -0.5, out=out), out, expect)


def test_token_contiguous_d512_graph_replays():
    g = torch.Generator().manual_seed(3)
    a = [torch.randn(1, 512, 1024, generator=g).half().to(DEV) for _ in range(3)]
    q, k, v = (t.transpose(1, 2).unsqueeze(1) for t in a)
    expect = gfx906_amd.attn(q, k, v, 512 ** -0.5)
    torch.cuda.synchronize()
    out = torch.empty_like(expect)
    replay_and_check(lambda: gfx906_amd.attn(q, k, v, 512 ** -0.5, out=out), out, expect)


def test_conv3d_graph_replays():
    g = torch.Generator().manual_seed(4)
    x = (torch.randn(1, 128, 4, 24, 24, generator=g) * 0.25).half().to(DEV).contiguous(
        memory_format=CL)
    w = (torch.randn(256, 128, 3, 3, 3, generator=g) * 0.25).half().to(DEV).contiguous(
        memory_format=CL)
    b = torch.randn(256, generator=g).half().to(DEV)
    expect = kitchen.try_kernel(x, w, b, None, [1, 1, 1])
    torch.cuda.synchronize()
    out = torch.empty_like(expect)
    replay_and_check(lambda: kitchen.try_kernel(x, w, b, None, [1, 1, 1], out=out), out, expect)
