"""CPU tests of the SDPA hook layer (gfx906_amd.attention_hooks), with fake host
modules in the manner of the reference's own test (test_vae_hook.py:11-68)."""

import sys
import types
from unittest import mock

import pytest
import torch

from gfx906_amd import attention_hooks as hooks
from gfx906_amd import loader


class FakeCuda:
    """Shape/dtype carrier that claims to live on a GPU."""

    is_cuda = True
    device = torch.device("cpu")  # where the hook allocates its output in these tests

    def __init__(self, shape, dtype=torch.float16):
        self.shape = torch.Size(shape)
        self.dtype = dtype
        self.ndim = len(shape)

    def dim(self):
        return self.ndim

    def reshape(self, *a):
        return self

    def transpose(self, *a):
        return self

    def unsqueeze(self, *a):
        return self


class Box:
    """Container with the peek()/take() protocol of the host's attention seam."""

    def __init__(self, t):
        self.t = t
        self.taken = False

    def peek(self):
        return self.t

    def take(self):
        self.taken = True
        return self.t


def fake_comfy(model=None, attention=None):
    names = ("comfy", "comfy.ldm", "comfy.ldm.modules", "comfy.ldm.modules.diffusionmodules",
             "comfy.ldm.modules.attention")
    mods = {n: types.ModuleType(n) for n in names}
    if model is not None:
        mods["comfy.ldm.modules.diffusionmodules"].model = model
        mods["comfy.ldm.modules.diffusionmodules.model"] = model
    if attention is not None:
        mods["comfy.ldm.modules"].attention = attention
        mods["comfy.ldm.modules.attention"] = attention
    return mods


# -- eligibility (reference deploy/gfx906_attention.py:38-49) ------------------------------

@pytest.mark.parametrize("d,ok", [(128, True), (512, True), (64, True), (8, True), (48, True),
                                  (72, False), (96, False), (256, False), (60, False)])
def test_head_dims(d, ok):
    q = FakeCuda((1, 4, 10, d))
    assert hooks.eligible(q, q, q, 4, None, {}) is ok


def test_eligibility_rejections():
    q = FakeCuda((2, 4, 10, 128))
    assert hooks.eligible(q, q, q, 4, None, {})
    assert not hooks.eligible(q, q, q, 4, object(), {})                      # mask
    assert not hooks.eligible(q, q, q, 4, None, {"enable_gqa": True})       # GQA
    assert not hooks.eligible(q, q, q, 8, None, {})                         # heads mismatch
    assert not hooks.eligible(FakeCuda((2, 4, 10, 128), torch.float32), q, q, 4, None, {})
    assert hooks.eligible(FakeCuda((2, 4, 10, 128), torch.bfloat16), q, q, 4, None, {})
    assert not hooks.eligible(q, FakeCuda((2, 4, 12, 128)), q, 4, None, {})  # k != v shape
    assert not hooks.eligible(q, FakeCuda((1, 4, 10, 128)), FakeCuda((1, 4, 10, 128)), 4, None,
                              {})                                            # batch mismatch
    assert not hooks.eligible(FakeCuda((2, 4, 10)), q, q, 4, None, {})       # not 4-D
    cpu = torch.zeros(2, 4, 10, 128, dtype=torch.float16)
    assert not hooks.eligible(cpu, cpu, cpu, 4, None, {})                    # not on the GPU


def test_decline_reasons_name_the_rule():
    q = FakeCuda((2, 4, 10, 128))
    assert hooks.decline_reason(q, q, q, 4, None, {}) is None
    assert hooks.decline_reason(q, q, q, 4, object(), {}) == "mask"
    assert hooks.decline_reason(q, q, q, 4, None, {"enable_gqa": True}) == "grouped-query attention"
    assert hooks.decline_reason(q, q, q, 2, None, {}) == "head count differs from `heads`"
    assert hooks.decline_reason(FakeCuda((2, 4, 10, 96)), FakeCuda((2, 4, 10, 96)),
                                FakeCuda((2, 4, 10, 96)), 4, None, {}) == "head dim 96"
    assert hooks.decline_reason(q, FakeCuda((2, 4, 10, 64)), FakeCuda((2, 4, 10, 64)), 4, None,
                                {}) == "q and k disagree on batch, heads or head dim"


# -- container function ------------------------------------------------------------------------

def test_container_ineligible_goes_to_stock():
    calls = []

    def stock(q, k, v, heads, **kw):
        calls.append((q, heads, kw))
        return "stock"

    q = torch.zeros(1, 2, 3, 128, dtype=torch.float16)  # CPU tensor: ineligible
    boxes = [Box(q), Box(q), Box(q)]
    with mock.patch.object(hooks.dit, "stock", stock):
        out = hooks.container_attn(*boxes, 2, skip_reshape=True, scale=0.5)
    assert out == "stock" and all(b.taken for b in boxes)
    assert calls[0][2]["skip_reshape"] is True and calls[0][2]["scale"] == 0.5


def test_container_requires_skip_reshape():
    called = []
    q = FakeCuda((1, 2, 3, 128))
    with mock.patch.object(hooks.dit, "stock", lambda *a, **k: called.append(1) or "s"), \
            mock.patch.object(loader, "load_attention", side_effect=AssertionError):
        assert hooks.container_attn(Box(q), Box(q), Box(q), 2, skip_reshape=False) == "s"
    assert called


def test_container_kernel_path_layout_and_bf16():
    """Kernel path with the op replaced by SDPA on CPU: bf16 reaches the op
    uncast, and the [B, S, H*D] result is the op's output written through an
    ``out`` view of a [B, S, H, D] buffer (no transpose copy afterwards)."""
    seen = []

    def fake_attn(q, k, v, scale, out=None):
        seen.append((q.dtype, scale, out))
        res = torch.nn.functional.scaled_dot_product_attention(
            q.float(), k.float(), v.float(), scale=scale).to(q.dtype)
        if out is None:
            return res
        out.copy_(res)
        return out

    mod = types.SimpleNamespace(attn=fake_attn)
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(2, 3, 5, 16, generator=g).bfloat16() for _ in range(3))
    with mock.patch.object(hooks, "eligible", return_value=True), \
            mock.patch.object(loader, "load_attention", return_value=mod):
        out = hooks.container_attn(Box(q), Box(k), Box(v), 3, skip_reshape=True)
        out_bhsd = hooks.container_attn(Box(q), Box(k), Box(v), 3, skip_reshape=True,
                                         skip_output_reshape=True, scale=0.3)
    (dt0, sc0, view), (dt1, sc1, none) = seen
    assert dt0 == dt1 == torch.bfloat16 and sc0 == 16 ** -0.5 and sc1 == 0.3 and none is None
    assert view.shape == (2, 3, 5, 16) and view.data_ptr() == out.data_ptr()
    assert out.dtype == torch.bfloat16 and out.shape == (2, 5, 3 * 16) and out.is_contiguous()
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float())
    torch.testing.assert_close(out.float(), ref.transpose(1, 2).reshape(2, 5, 48), atol=2e-2,
                               rtol=0)
    assert out_bhsd.shape == (2, 3, 5, 16)


def test_container_kernel_error_falls_back_to_stock():
    """A call the kernel raises on (e.g. a size it rejects) runs on the stock
    path with the original arguments."""
    stock_calls = []

    def stock(q, k, v, heads, **kw):
        stock_calls.append((q, heads, kw))
        return "stock"

    mod = types.SimpleNamespace(attn=mock.Mock(side_effect=RuntimeError("kernel: too large")))
    q = torch.zeros(1, 2, 3, 128, dtype=torch.float16)
    with mock.patch.object(hooks, "eligible", return_value=True), \
            mock.patch.object(loader, "load_attention", return_value=mod), \
            mock.patch.object(hooks.dit, "stock", stock):
        assert hooks.container_attn(Box(q), Box(q), Box(q), 2, skip_reshape=True,
                                    scale=0.25) == "stock"
    mod.attn.assert_called_once()
    assert stock_calls[0][0] is q and stock_calls[0][2]["scale"] == 0.25


# -- VAE hook (reference test_vae_hook.py:11-68) -------------------------------------------

def test_vae_factory_preserves_selected_fallback():
    def normal(q, k, v):
        return "normal"

    def pytorch(q, k, v):
        return "pytorch"

    def other(q, k, v):
        return "other"

    for selected in (normal, pytorch, other):
        model = types.SimpleNamespace(normal_attention=normal, pytorch_attention=pytorch,
                                      vae_attention=lambda s=selected: s)
        with mock.patch.dict(sys.modules, fake_comfy(model=model)), \
                mock.patch.object(hooks.vae, "model", None):
            hooks.install_vae_hook()
            fn = model.vae_attention()
            if selected is other:
                assert fn is other
            # CPU tensor -> ineligible -> the selected function runs
            assert fn(torch.zeros(1), None, None) == selected(None, None, None)


def test_vae_kernel_error_uses_selected_fallback():
    t = FakeCuda((1, 512, 2, 2))
    kernel = types.SimpleNamespace(attn=mock.Mock(side_effect=RuntimeError))
    with mock.patch.object(loader, "load_attention", return_value=kernel):
        assert hooks.vae_attn(t, t, t, lambda q, k, v: "fallback") == "fallback"
    kernel.attn.assert_called_once()


def test_vae_writes_nchw_output_in_place():
    # q/k/v [b, c, h, w] -> token-contiguous [b, 1, h*w, c] views (sequence stride
    # 1, channel stride h*w); the kernel writes a view of the returned tensor.
    b, c, h, w = 2, 512, 3, 5
    q, k, v = (torch.randn(b, c, h, w).half() for _ in range(3))
    seen = {}

    def fake_attn(qt, kt, vt, scale, out=None):
        seen.update(q=qt, k=kt, scale=scale, out=out)
        out.copy_(qt * 2)  # any function of the inputs, written through the view
        return out

    kernel = types.SimpleNamespace(attn=fake_attn)
    with mock.patch.object(loader, "load_attention", return_value=kernel), \
            mock.patch.object(torch.Tensor, "is_cuda", new_callable=mock.PropertyMock,
                              return_value=True):
        res = hooks.vae_attn(q, k, v, lambda *a: "fallback")
    assert seen["scale"] == c ** -0.5
    for name in ("q", "k", "out"):
        t = seen[name]
        assert t.shape == (b, 1, h * w, c) and t.stride(2) == 1 and t.stride(3) == h * w
    assert seen["q"].data_ptr() == q.data_ptr()  # no copy of the input
    assert res.shape == (b, c, h, w) and res.is_contiguous()
    assert seen["out"].data_ptr() == res.data_ptr()
    assert torch.equal(res, q * 2)


def test_vae_ineligible_channels_use_fallback():
    t = FakeCuda((1, 256, 2, 2))
    with mock.patch.object(loader, "load_attention", side_effect=AssertionError):
        assert hooks.vae_attn(t, t, t, lambda q, k, v: "fallback") == "fallback"


# -- install --------------------------------------------------------------------------------------

def test_install_is_noop_off_gfx950():
    with mock.patch.object(loader, "is_gfx950", return_value=False), \
            mock.patch.dict(sys.modules, {"comfy": None}):
        hooks.install()  # must not try to import the host application


def test_install_sets_container_function_once():
    opt = types.SimpleNamespace(container_function=None)
    attention = types.SimpleNamespace(optimized_attention=opt)
    with mock.patch.object(loader, "is_gfx950", return_value=True), \
            mock.patch.dict(sys.modules, fake_comfy(attention=attention)), \
            mock.patch.object(hooks.dit, "stock", None):
        hooks.install()
        assert opt.container_function is hooks.container_attn
        assert hooks.dit.stock is opt
        hooks.install()  # second call: no change
        assert opt.container_function is hooks.container_attn


def test_install_leaves_existing_container_function():
    sentinel = object()
    opt = types.SimpleNamespace(container_function=sentinel)
    attention = types.SimpleNamespace(optimized_attention=opt)
    with mock.patch.object(loader, "is_gfx950", return_value=True), \
            mock.patch.dict(sys.modules, fake_comfy(attention=attention)), \
            mock.patch.object(hooks.dit, "stock", None):
        hooks.install()
    assert opt.container_function is sentinel
