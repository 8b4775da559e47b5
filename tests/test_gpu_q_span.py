"""Query tiles whose rows span 2 GiB or more: the predicated Q load.

The D <= 128 ring kernels (Q in registers: up to 1024 keys at D <= 64, 256 at
D = 128, and every padded head dim) and the D = 512 kernel with row-major K/V
load a workgroup's Q rows through one range-checked buffer descriptor when
the rows span less than 2 GiB (sequence stride below about 4.2 M elements at
256 rows per workgroup, 8.4 M at 128), and row by row with predicated global
loads otherwise. Each case here gives Q a sequence stride past that bound
(heads interleaved in each row, Sq ragged against the workgroup rows) and
checks, for a positive and a negative scale, that

* the output equals, bit for bit, the same call with a contiguous Q (which
  takes the descriptor path),
* seeded rows meet the parity bar against SDPA MATH in fp32 on the CPU.

Each case prints its parameters first.
"""

import pytest
import torch

import gfx906_amd
from oracle.attention import MAX_ABS_TOL, MEAN_ABS_TOL, error_stats, make_inputs, sdpa_math_fp32

pytestmark = pytest.mark.gpu

# sequence strides (elements) just past the 2 GiB span of 256 and 128 rows
STRIDE_256 = (1 << 31) // (255 * 2) + 4096
STRIDE_128 = (1 << 31) // (127 * 2) + 4096
CASES = [  # B, H, Sq, Skv, D, sequence stride of q
    (1, 2, 300, 300, 64, STRIDE_256),  # D = 64, keys <= 1024: Q in registers
    (1, 2, 300, 200, 128, STRIDE_256),  # D = 128, keys <= 256: Q in registers
    (1, 2, 270, 500, 40, STRIDE_256),  # padded head dim
    (1, 2, 130, 100, 512, STRIDE_128),  # D = 512, row-major K/V
]


@pytest.fixture(scope="module")
def qbuf():
    need = max((Sq - 1) * s + H * D for _, H, Sq, _, D, s in CASES)
    if torch.cuda.mem_get_info()[0] < 2 * need + (4 << 30):
        pytest.skip("not enough free device memory for a 3 GiB query buffer")
    buf = torch.empty(need, dtype=torch.float16, device="cuda")
    yield buf
    del buf
    torch.cuda.empty_cache()


@pytest.mark.parametrize("sign", [1.0, -1.0])
@pytest.mark.parametrize("B,H,Sq,Skv,D,stride", CASES)
def test_q_rows_span_past_2gib(qbuf, B, H, Sq, Skv, D, stride, sign):
    print(f"case: B{B} H{H} Sq{Sq} Skv{Skv} D{D} q sequence stride {stride} sign {sign}",
          flush=True)
    assert (255 if D <= 128 else 127) * stride * 2 + 2 * max(D, 64) >= (1 << 31)
    q, k, v = make_inputs(B, H, Sq, Skv, D, 1.0, 1.0, 23)
    scale = sign * D ** -0.5
    qc, kc, vc = (t.cuda() for t in (q, k, v))
    qw = qbuf[: (Sq - 1) * stride + H * D].as_strided((B, H, Sq, D), (0, D, stride, 1))
    qw.copy_(qc)
    wide = gfx906_amd.attn(qw, kc, vc, scale)
    near = gfx906_amd.attn(qc, kc, vc, scale)
    torch.cuda.synchronize()
    assert torch.isfinite(wide).all()
    assert torch.equal(wide, near)
    rows = torch.cat([torch.arange(64), torch.arange(Sq - 64, Sq)])
    ref = sdpa_math_fp32(q[:, :, rows], k, v, scale)
    mx, mn = error_stats(wide[:, :, rows.cuda()].float().cpu(), ref)
    print(f"  wide == contiguous; {len(rows)} rows per head: max-abs {mx:.3e} "
          f"mean-abs {mn:.3e}", flush=True)
    assert mx <= MAX_ABS_TOL and mn <= MEAN_ABS_TOL
