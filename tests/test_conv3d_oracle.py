"""Pins the conv3d oracle (oracle/conv3d.py) on the CPU: against torch's conv3d
in fp64 (library routine), brute-force loops, and the layout identities the
kernels rely on. Planted mistakes must fail the same checks."""

import numpy as np
import pytest
import torch

from oracle import conv3d as oc


def torch_ref(x, w, bias, res, stride):
    o = torch.nn.functional.conv3d(torch.from_numpy(x).double(), torch.from_numpy(w).double(),
                                   None if bias is None else torch.from_numpy(bias).double(),
                                   stride=stride)
    if res is not None:
        o = o + torch.from_numpy(res).double()
    return o.numpy()


@pytest.mark.parametrize("xs,ws,stride,b,r", [
    ((1, 8, 3, 6, 5), (8, 3, 3, 3), (1, 1, 1), True, True),
    ((2, 16, 5, 7, 9), (24, 3, 2, 3), (2, 1, 2), True, False),
    ((1, 8, 4, 4, 4), (16, 1, 1, 1), (1, 1, 1), False, True),
    ((1, 24, 3, 9, 9), (8, 1, 3, 3), (1, 2, 2), True, True),
    ((2, 8, 6, 5, 5), (8, 3, 3, 3), (3, 2, 1), False, False),
])
def test_gemm_matches_torch_conv3d(xs, ws, stride, b, r):
    x, w, bias, res = oc.make_case(xs, ws, stride, b, r, seed=sum(xs) + sum(ws))
    got = oc.conv3d_gemm(x, w, bias, res, stride)
    np.testing.assert_allclose(got, torch_ref(x, w, bias, res, stride), rtol=0, atol=1e-9)


def test_gemm_matches_brute_force():
    x, w, bias, res = oc.make_case((1, 8, 3, 4, 4), (8, 2, 3, 2), (1, 1, 2), True, True, seed=7)
    np.testing.assert_allclose(oc.conv3d_gemm(x, w, bias, res, (1, 1, 2)),
                               oc.conv3d_brute(x, w, bias, res, (1, 1, 2)), rtol=0, atol=1e-9)


def test_weight_rows_is_channels_last_3d_memory():
    # The kernels read w[k] as one contiguous [KG] row: that is what a packed
    # channels_last_3d [K, C, T, R, S] tensor holds in memory.
    _, w, _, _ = oc.make_case((1, 16, 3, 3, 3), (8, 3, 2, 3), (1, 1, 1), False, False, seed=3)
    t = torch.from_numpy(w).contiguous(memory_format=torch.channels_last_3d)
    flat = torch.as_strided(t, (t.numel(),), (1,)).numpy().reshape(8, -1)
    np.testing.assert_array_equal(flat, oc.weight_rows(w))


def test_reduction_order_groups_of_8_stay_in_one_tap():
    # With C % 8 == 0 every aligned 8-element group of i has one (t, r, s).
    C, T, R, S = 24, 2, 3, 2
    i = np.arange(C * T * R * S)
    tap = i // C
    assert all(len(set(tap[g:g + 8])) == 1 for g in range(0, len(i), 8))


def test_fp16_output_is_rne_of_gemm():
    x, w, bias, res = oc.make_case((1, 8, 3, 5, 5), (8, 3, 3, 3), (1, 1, 1), True, True, seed=9)
    g = oc.conv3d_gemm(x, w, bias, res)
    o = oc.conv3d_fp16(x, w, bias, res)
    assert o.dtype == np.float16
    np.testing.assert_array_equal(o, torch.from_numpy(g).to(torch.float16).numpy())


def test_output_size():
    assert oc.output_size(4, 32, 32, 3, 3, 3, (1, 1, 1)) == (2, 30, 30)
    assert oc.output_size(6, 16, 16, 3, 3, 3, (2, 1, 1)) == (2, 14, 14)
    assert oc.output_size(4, 32, 32, 3, 3, 3, (1, 2, 2)) == (2, 15, 15)


@pytest.mark.parametrize("mistake", ["swap_tr", "drop_bias", "h_off_by_one", "res_sign"])
def test_planted_mistakes_are_caught(mistake):
    xs, ws, stride = (1, 8, 4, 5, 6), (8, 2, 3, 2), (1, 2, 1)
    x, w, bias, res = oc.make_case(xs, ws, stride, True, True, seed=11)
    ref = torch_ref(x, w, bias, res, stride)
    if mistake == "swap_tr":  # reduction index with r and t exchanged
        bad = oc.conv3d_gemm(x, np.ascontiguousarray(np.swapaxes(w, 2, 3)).reshape(w.shape),
                             bias, res, stride)
    elif mistake == "drop_bias":
        bad = oc.conv3d_gemm(x, w, None, res, stride)
    elif mistake == "h_off_by_one":  # window rows read one row late
        bad = oc.conv3d_gemm(x[:, :, :, 1:, :], w, bias, None, (1, 2, 1))
        bad = bad[..., :ref.shape[3], :] if bad.shape[3] >= ref.shape[3] else bad
        bad = bad + res[..., :bad.shape[3], :]
        ref = ref[..., :bad.shape[3], :]
    else:
        bad = oc.conv3d_gemm(x, w, bias, -res, stride)
    assert np.abs(bad - ref).max() > 1e-3


def test_reference_cases_are_valid_shapes():
    for xs, ws, stride, b, r in oc.REF_CASES:
        n, c, d, h, w = xs
        k, t, rr, s = ws
        assert c % 8 == 0 and k % 8 == 0
        assert min(oc.output_size(d, h, w, t, rr, s, stride)) > 0
