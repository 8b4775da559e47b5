"""CPU oracle for the conv3d path: test infrastructure only.

Imported by tests/ only; the product (gfx906_amd/) never imports it.

Restates the reference's fp16 conv3d contract (hip_conv/conv3d_kernel.hip:8-13
GEMM view, :171-215 epilogue; gfx906_kitchen.py:167-227 shapes and layouts):

    out[n,k,z,p,q] = fp16( sum_{c,t,r,s} x[n,c,z*sd+t,p*sh+r,q*sw+s] * w[k,c,t,r,s]
                           + bias[k] + res[n,k,z,p,q] )

as the implicit GEMM the kernels run: rows m = ((n*Z + z)*P + p)*Q + q,
columns k, reduction index i = ((t*R + r)*S + s)*C + c. Accumulation is fp64
here (the kernels accumulate in fp32; the difference is far below the fp16
output rounding).

Pinned in tests/test_conv3d_oracle.py against torch.nn.functional.conv3d in
fp64 (library routine), brute-force loops on tiny shapes, and the layout
identity the kernels rely on (a packed channels_last_3d weight is the [K, KG]
GEMM operand in memory order).
"""

from __future__ import annotations

import numpy as np


def output_size(d, h, w, t, r, s, stride):
    """(Z, P, Q) of a VALID convolution (gfx906_kitchen.py:175)."""
    sd, sh, sw = stride
    return (d - t) // sd + 1, (h - r) // sh + 1, (w - s) // sw + 1


def weight_rows(w):
    """[K, C, T, R, S] -> [K, KG] with column i = ((t*R + r)*S + s)*C + c
    (conv3d_kernel.hip:10-13)."""
    k, c, t, r, s = w.shape
    return np.ascontiguousarray(np.transpose(w, (0, 2, 3, 4, 1))).reshape(k, t * r * s * c)


def im2col(x, t, r, s, stride):
    """[N, C, D, H, W] -> [M, KG]: row m = ((n*Z + z)*P + p)*Q + q holds the
    window of output voxel (n, z, p, q) in reduction order (t, r, s, c)."""
    n, c, d, h, w = x.shape
    sd, sh, sw = stride
    Z, P, Q = output_size(d, h, w, t, r, s, stride)
    cols = np.empty((n, Z, P, Q, t, r, s, c), dtype=np.float64)
    xf = x.astype(np.float64)
    for dt in range(t):
        for dr in range(r):
            for ds in range(s):
                win = xf[:, :, dt:dt + (Z - 1) * sd + 1:sd, dr:dr + (P - 1) * sh + 1:sh,
                         ds:ds + (Q - 1) * sw + 1:sw]  # [N, C, Z, P, Q]
                cols[:, :, :, :, dt, dr, ds, :] = np.transpose(win, (0, 2, 3, 4, 1))
    return cols.reshape(n * Z * P * Q, t * r * s * c)


def conv3d_gemm(x, w, bias=None, res=None, stride=(1, 1, 1)):
    """fp64 [N, K, Z, P, Q] result of the implicit GEMM plus bias and residual,
    before the output rounding."""
    n, c, d, h, wd = x.shape
    k, cw, t, r, s = w.shape
    assert cw == c
    Z, P, Q = output_size(d, h, wd, t, r, s, stride)
    o = im2col(x, t, r, s, stride) @ weight_rows(w).astype(np.float64).T  # [M, K]
    if bias is not None:
        o = o + np.asarray(bias, dtype=np.float64)[None, :]
    o = o.reshape(n, Z, P, Q, k).transpose(0, 4, 1, 2, 3)
    if res is not None:
        o = o + np.asarray(res, dtype=np.float64)
    return o


def conv3d_fp16(x, w, bias=None, res=None, stride=(1, 1, 1)):
    """conv3d_gemm rounded to fp16 (round to nearest even), the kernels' output."""
    return conv3d_gemm(x, w, bias, res, stride).astype(np.float16)


def conv3d_brute(x, w, bias=None, res=None, stride=(1, 1, 1)):
    """Direct six-deep loops over the definition (tiny shapes only)."""
    n, c, d, h, wd = x.shape
    k, _, t, r, s = w.shape
    sd, sh, sw = stride
    Z, P, Q = output_size(d, h, wd, t, r, s, stride)
    out = np.zeros((n, k, Z, P, Q), dtype=np.float64)
    for nn in range(n):
        for kk in range(k):
            for z in range(Z):
                for p in range(P):
                    for q in range(Q):
                        acc = 0.0
                        for cc in range(c):
                            for dt in range(t):
                                for dr in range(r):
                                    for ds in range(s):
                                        acc += (float(x[nn, cc, z * sd + dt, p * sh + dr, q * sw + ds])
                                                * float(w[kk, cc, dt, dr, ds]))
                        if bias is not None:
                            acc += float(bias[kk])
                        if res is not None:
                            acc += float(res[nn, kk, z, p, q])
                        out[nn, kk, z, p, q] = acc
    return out


# The reference's own GPU check cases (test_conv3d.py:58-69):
# (n, c, d, h, w), (k, t, r, s), stride, bias, residual
REF_CASES = [
    ((1, 128, 4, 32, 32), (256, 3, 3, 3), (1, 1, 1), True, True),
    ((1, 256, 4, 32, 32), (128, 3, 3, 3), (1, 1, 1), True, False),
    ((1, 512, 4, 16, 16), (512, 3, 3, 3), (1, 1, 1), False, True),
    ((1, 128, 5, 33, 17), (64, 3, 3, 3), (1, 1, 1), True, True),
    ((1, 128, 8, 32, 32), (128, 1, 1, 1), (1, 1, 1), True, False),
    ((1, 64, 6, 16, 16), (64, 3, 3, 3), (2, 1, 1), True, True),
    ((1, 96, 4, 32, 32), (96, 3, 3, 3), (1, 2, 2), True, False),
    ((1, 8, 3, 16, 16), (8, 3, 3, 3), (1, 1, 1), True, True),
    ((2, 64, 3, 16, 16), (64, 3, 3, 3), (1, 1, 1), True, True),
    ((1, 128, 1, 32, 32), (256, 1, 3, 3), (1, 1, 1), True, True),
]


def make_case(xs, ws, stride, has_bias, has_res, seed):
    """fp16 numpy inputs of one case: x, w ~ 0.25*N(0,1), bias ~ N(0,1),
    residual ~ 0.25*N(0,1) (the scales of test_conv3d.py:53-55, 69-73)."""
    rng = np.random.default_rng(seed)
    n, c, d, h, w = xs
    k, t, r, s = ws
    x = (rng.standard_normal(xs) * 0.25).astype(np.float16)
    wt = (rng.standard_normal((k, c, t, r, s)) * 0.25).astype(np.float16)
    b = rng.standard_normal(k).astype(np.float16) if has_bias else None
    Z, P, Q = output_size(d, h, w, t, r, s, stride)
    res = (rng.standard_normal((n, k, Z, P, Q)) * 0.25).astype(np.float16) if has_res else None
    return x, wt, b, res
