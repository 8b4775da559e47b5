"""CPU tests of the conv3d backend layer (gfx906_amd.kitchen): layout helpers,
the arguments handed to the kernel op, the decline rules and the torch
fallback (reference contract: gfx906_kitchen.py:114-248), and registration
into a fake comfy_kitchen registry (gfx906_kitchen.py:255-299)."""

import sys
import types
from unittest import mock

import pytest
import torch

from gfx906_amd import kitchen

CL = torch.channels_last_3d


class FakeExt:
    def __init__(self):
        self.calls = []

    def conv3d(self, x, w, bias, res, out, dims, xs, os, rs):
        self.calls.append(dict(x=x, w=w, bias=bias, res=res, out=out, dims=dims, xs=xs, os=os,
                               rs=rs))


@pytest.fixture
def fake_ext():
    ext = FakeExt()
    with mock.patch.object(kitchen, "load", return_value=ext), \
            mock.patch.object(torch.Tensor, "is_cuda", new_callable=mock.PropertyMock,
                              return_value=True):
        yield ext


def cl(shape, dtype=torch.float16):
    return torch.zeros(shape, dtype=dtype).contiguous(memory_format=CL)


# -- layout helpers ---------------------------------------------------------------------------

def test_ndhwc_strides():
    x = cl((2, 16, 3, 5, 7))
    assert kitchen.ndhwc_strides(x) == (3 * 5 * 7 * 16, 5 * 7 * 16, 7 * 16, 16)
    assert kitchen.ndhwc_strides(x[:, :, 1:3]) == (3 * 5 * 7 * 16, 5 * 7 * 16, 7 * 16, 16)
    assert kitchen.ndhwc_strides(torch.zeros(2, 16, 3, 5, 7)) is None        # NCDHW
    assert kitchen.ndhwc_strides(cl((1, 4, 3, 5, 7))) is None                 # C=4: strides % 8
    assert kitchen.ndhwc_strides(torch.zeros(2, 16, 3, 5)) is None            # not 5-D
    assert kitchen.packed_strides((2, 16, 3, 5, 7)) == (3 * 5 * 7 * 16, 5 * 7 * 16, 7 * 16, 16)


def test_tensors_overlap():
    buf = torch.zeros(100)
    assert kitchen.may_overlap(buf[0:10], buf[5:15])
    assert not kitchen.may_overlap(buf[0:10], buf[10:20])
    assert not kitchen.may_overlap(buf, torch.zeros(100))
    assert kitchen.may_overlap(buf[::2], buf[1::2])  # interleaved: extents intersect


# -- arguments passed to the op ----------------------------------------------------------------

def test_packed_inputs_bias_residual(fake_ext):
    x, w = cl((2, 16, 5, 6, 7)), cl((24, 16, 3, 3, 3))
    b = torch.zeros(24, dtype=torch.float16)
    res = cl((2, 24, 3, 4, 5))
    out = kitchen.try_kernel(x, w, b, res, [1, 1, 1])
    (c,) = fake_ext.calls
    assert c["dims"] == [2, 5, 6, 7, 16, 24, 3, 3, 3, 1, 1, 1, 3, 4, 5]
    assert c["xs"] == list(kitchen.packed_strides(x.shape))
    assert c["os"] == list(kitchen.packed_strides(out.shape)) == c["rs"]
    assert out.shape == (2, 24, 3, 4, 5) and out.is_contiguous(memory_format=CL)
    assert c["out"] is out and c["res"] is res


def test_ncdhw_input_converted_and_strided_output(fake_ext):
    x, w = torch.zeros(1, 16, 4, 9, 9, dtype=torch.float16), cl((8, 16, 1, 3, 3))
    big = cl((1, 8, 10, 4, 4))
    out = big[:, :, 2:6]
    got = kitchen.try_kernel(x, w, None, None, (1, 2, 2), out=out)
    (c,) = fake_ext.calls
    assert got is out and c["x"].is_contiguous(memory_format=CL)
    assert c["dims"][12:] == [4, 4, 4]
    assert c["os"] == [10 * 4 * 4 * 8, 4 * 4 * 8, 4 * 8, 8] and c["rs"] == [0, 0, 0, 0]


def test_residual_may_be_out(fake_ext):
    x, w = cl((1, 8, 3, 6, 6)), cl((8, 8, 1, 3, 3))
    out = cl((1, 8, 3, 4, 4))
    assert kitchen.try_kernel(x, w, None, out, (1, 1, 1), out=out) is out
    assert fake_ext.calls[0]["res"] is out


@pytest.mark.parametrize("case", ["C", "K", "dtype", "bias_shape", "res_shape", "taps",
                                  "stride0", "too_small", "out_overlaps_x", "out_batch0"])
def test_declines(fake_ext, case):
    x, w, b, res, stride, out = cl((2, 16, 5, 6, 7)), cl((24, 16, 3, 3, 3)), None, None, (1, 1, 1), None
    if case == "C":
        x, w = cl((2, 12, 5, 6, 7)), cl((24, 12, 3, 3, 3))
    elif case == "K":
        w = cl((20, 16, 3, 3, 3))
    elif case == "dtype":
        x = x.float()
    elif case == "bias_shape":
        b = torch.zeros(23, dtype=torch.float16)
    elif case == "res_shape":
        res = cl((2, 24, 3, 4, 4))
    elif case == "taps":
        x, w = cl((1, 8, 11, 11, 11)), cl((8, 8, 11, 11, 11))  # 1331 taps
    elif case == "stride0":
        stride = (1, 0, 1)
    elif case == "too_small":
        x = cl((2, 16, 2, 6, 7))
    elif case == "out_overlaps_x":
        big = cl((2, 24, 5, 6, 7))
        x = big[:, :16]
        out = big[:, :24, :3, :4, :5]
    elif case == "out_batch0":
        out = cl((1, 24, 3, 4, 5)).expand(2, 24, 3, 4, 5)
    assert kitchen.try_kernel(x, w, b, res, stride, out=out) is None
    assert not fake_ext.calls


def test_plan_names_decline_reasons(fake_ext):
    x, w = cl((2, 16, 5, 6, 7)), cl((24, 16, 3, 3, 3))
    assert isinstance(kitchen.plan(x, w, None, None, (1, 1, 1)), kitchen.ConvCall)
    assert kitchen.plan(x, cl((20, 16, 3, 3, 3)), None, None, (1, 1, 1)) == \
        "C and K must be positive multiples of 8"
    assert kitchen.plan(x, w, None, None, (1, 0, 1)) == "stride below 1"
    assert kitchen.plan(cl((2, 16, 2, 6, 7)), w, None, None, (1, 1, 1)) == \
        "input smaller than the filter"
    big = cl((2, 24, 5, 6, 7))
    assert kitchen.plan(big[:, :16], w, None, None, (1, 1, 1), out=big[:, :24, :3, :4, :5]) == \
        "out shares memory with an input"
    assert not fake_ext.calls


def test_bad_out_raises(fake_ext):
    with pytest.raises(ValueError):
        kitchen.try_kernel(cl((1, 8, 3, 6, 6)), cl((8, 8, 1, 3, 3)), None, None, (1, 1, 1),
                             out=cl((1, 8, 3, 4, 5)))


# -- fallback and registration -------------------------------------------------------------

def test_fallback_is_torch_conv_plus_residual():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, 8, 3, 6, 6, generator=g).half().contiguous(memory_format=CL)
    w = torch.randn(8, 8, 1, 3, 3, generator=g).half()
    b = torch.randn(8, generator=g).half()
    res = torch.randn(1, 8, 3, 4, 4, generator=g).half()
    with mock.patch.object(kitchen, "load", return_value=None):
        out = kitchen.fp16_conv3d(x, w, b, res, [1, 1, 1])
        into = torch.empty(1, 8, 3, 4, 4, dtype=torch.float16)
        kitchen.fp16_conv3d_out(x, w, b, res, [1, 1, 1], into)
    ref = torch.nn.functional.conv3d(x, w, b) + res
    assert torch.equal(out, ref) and out.is_contiguous(memory_format=CL)
    assert torch.equal(into, ref)


def fake_kitchen_modules(registry):
    ck = types.ModuleType("comfy_kitchen")
    reg = types.ModuleType("comfy_kitchen.registry")
    reg.registry = registry
    cons = types.ModuleType("comfy_kitchen.constraints")

    class Rec:
        def __init__(self, *a, **k):
            self.a, self.k = a, k

    cons.ExactDims = cons.FunctionConstraints = cons.ParamConstraint = Rec
    cons.with_out_param = lambda c: ("out", c)
    return {"comfy_kitchen": ck, "comfy_kitchen.registry": reg, "comfy_kitchen.constraints": cons}


class FakeRegistry:
    def __init__(self):
        self._priority = ["cuda", "eager"]
        self.registered = {}

    def register(self, name, module, caps):
        self.registered[name] = (module, caps)

    def set_priority(self, order):
        self._priority = list(order)


def test_install_registers_first(monkeypatch):
    reg = FakeRegistry()
    monkeypatch.setenv("GFX906_AMD_KITCHEN_FORCE", "1")
    with mock.patch.dict(sys.modules, fake_kitchen_modules(reg)), \
            mock.patch.object(kitchen, "load", return_value=FakeExt()):
        assert kitchen.install()
    module, caps = reg.registered["gfx950"]
    assert module is kitchen and set(caps) == {"fp16_conv3d", "fp16_conv3d_out"}
    assert reg._priority == ["gfx950", "cuda", "eager"]


def test_install_noop_off_gfx950_or_without_kitchen(monkeypatch):
    monkeypatch.delenv("GFX906_AMD_KITCHEN_FORCE", raising=False)
    monkeypatch.delenv("GFX906_KITCHEN_FORCE", raising=False)
    with mock.patch.object(kitchen, "is_gfx950", return_value=False):
        assert not kitchen.install()
    monkeypatch.setenv("GFX906_KITCHEN_FORCE", "1")
    with mock.patch.dict(sys.modules, {"comfy_kitchen": None, "comfy_kitchen.registry": None}):
        assert not kitchen.install()
    reg = FakeRegistry()
    with mock.patch.dict(sys.modules, fake_kitchen_modules(reg)), \
            mock.patch.object(kitchen, "load", return_value=None):
        assert not kitchen.install() and not reg.registered
