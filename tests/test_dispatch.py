"""The import surface and routing of amd_tuned_torch on the CPU (no GPU, native layer
mocked where a call must reach it): enable()/disable(), the F.conv1d wrapper installed
at import, config 1 (a depthwise conv1d on CPU tensors goes to stock bit-exactly), the
conv/GroupNorm routing decisions and contests, the GroupNorm+SiLU Sequential fusion, and
the autograd wrappers' backward passes."""
from __future__ import annotations

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

import amd_tuned_torch as att
from amd_tuned_torch import _dispatch, _native, conv_fusion_ops, kernel_select, miopen_fallback

STOCK_CONV1D = miopen_fallback._original_conv1d


# ---------------------------------------------------------------------------
# install / restore
# ---------------------------------------------------------------------------
def test_autopatch_at_import_and_conv1d_wrapper():
    assert att.is_enabled()
    assert F.conv2d is _dispatch._patched_conv2d
    assert F.conv3d is _dispatch._patched_conv3d
    assert F.group_norm is _dispatch._patched_group_norm
    assert miopen_fallback.is_conv1d_fallback_enabled()
    assert F.conv1d is not STOCK_CONV1D


def test_enable_disable_idempotent_and_restores():
    originals = {name: fn for (tgt, name), fn in _dispatch._ORIGINALS.items() if tgt is F}
    att.enable()
    att.enable()
    assert F.group_norm is _dispatch._patched_group_norm
    att.disable()
    try:
        assert not att.is_enabled()
        for name, fn in originals.items():
            assert getattr(F, name) is fn
        # the conv1d wrapper is independent of enable()/disable() (reference behaviour)
        assert miopen_fallback.is_conv1d_fallback_enabled()
    finally:
        att.enable()
    assert F.group_norm is _dispatch._patched_group_norm


def test_conv1d_fallback_toggle():
    miopen_fallback.disable_conv1d_fallback()
    try:
        assert F.conv1d is STOCK_CONV1D
        assert not miopen_fallback.is_conv1d_fallback_enabled()
    finally:
        miopen_fallback.enable_conv1d_fallback()
    assert miopen_fallback.is_conv1d_fallback_enabled()


def test_config1_cpu_depthwise_conv1d_is_bit_exact_stock():
    """N=8, C=256, L=2048, k=3, pad 1, groups=C, bias, fp32, seeded, on
    the CPU with the package imported: routed to stock, bit-identical."""
    g = torch.Generator().manual_seed(1001)
    x = torch.randn(8, 256, 2048, generator=g)
    w = torch.randn(256, 1, 3, generator=g) * (1 / 3) ** 0.5
    b = torch.randn(256, generator=g) * 0.1 ** 0.5
    y = F.conv1d(x, w, b, padding=1, groups=256)
    assert torch.equal(y, STOCK_CONV1D(x, w, b, 1, 1, 1, 256))
    assert kernel_select.debug_winners() == {} or all(k[0] != "conv1d" for k in kernel_select.debug_winners())


def test_cpu_tensors_go_to_stock_for_every_patched_op():
    g = torch.Generator().manual_seed(0)
    x2, w2 = torch.randn(1, 3, 8, 8, generator=g), torch.randn(4, 3, 3, 3, generator=g)
    x3, w3 = torch.randn(1, 3, 4, 5, 6, generator=g), torch.randn(4, 3, 3, 3, 3, generator=g)
    xg = torch.randn(2, 8, 5, 5, generator=g)
    orig = _dispatch._ORIGINALS
    assert torch.equal(F.conv2d(x2, w2, None, 1, 1), orig[(F, "conv2d")](x2, w2, None, 1, 1))
    assert torch.equal(F.conv3d(x3, w3, None, 1, 1), orig[(F, "conv3d")](x3, w3, None, 1, 1))
    assert torch.equal(F.group_norm(xg, 4), orig[(F, "group_norm")](xg, 4))
    assert torch.equal(att.group_norm_silu(xg, 4), F.silu(orig[(F, "group_norm")](xg, 4)))


# ---------------------------------------------------------------------------
# routing with the native layer mocked
# ---------------------------------------------------------------------------
class FakeNative:
    """Stands in for the ctypes layer: records calls and computes with stock CPU ops."""

    def __init__(self, monkeypatch, conv_variants, gn_variants, decline=()):
        self.calls = []
        self.decline = set(decline)
        orig = _dispatch._ORIGINALS
        conv_names = ["direct"] + list(conv_variants)

        def conv(nd):
            def fn(input, weight, bias=None, stride=1, padding=0, dilation=1, *, variant=-1, out=None):
                name = conv_names[variant]
                self.calls.append((f"conv{nd}d", name))
                if name in self.decline:
                    raise _native.Unsupported("declined")
                return orig[(F, f"conv{nd}d")](input, weight, bias, stride, padding, dilation)
            return fn

        def gn(input, num_groups, weight=None, bias=None, eps=1e-5, *, silu=False, variant=-1, out=None):
            name = gn_variants[variant]
            self.calls.append(("group_norm", name))
            if name in self.decline:
                raise _native.Unsupported("declined")
            y = orig[(F, "group_norm")](input, num_groups, weight, bias, eps)
            return F.silu(y) if silu else y

        def variants(op):
            return {_native.OP_CONV: conv_names, _native.OP_GROUP_NORM: list(gn_variants),
                    _native.OP_DWCONV1D: ["lds_opt16"]}[op]

        def to_contiguous(x):
            self.calls.append(("layout", "to_ncdhw"))
            return x.contiguous()

        def to_channels_last(x):
            self.calls.append(("layout", "to_channels_last"))
            return x.contiguous(memory_format=torch.channels_last if x.dim() == 4 else torch.channels_last_3d)

        monkeypatch.setattr(_native, "conv2d", conv(2))
        monkeypatch.setattr(_native, "conv3d", conv(3))
        monkeypatch.setattr(_native, "group_norm", gn)
        monkeypatch.setattr(_native, "variants", variants)
        monkeypatch.setattr(_native, "channels_last_to_contiguous", to_contiguous)
        monkeypatch.setattr(_native, "contiguous_to_channels_last", to_channels_last)
        monkeypatch.setattr(_native, "available", lambda: True)
        monkeypatch.setattr(_dispatch, "_variant_cache", {})
        # everything _usable checks except the device (these are CPU tensors)
        monkeypatch.setattr(_dispatch, "_usable", lambda *t, dtypes=_dispatch._CONV_NATIVE_DTYPES: all(
            type(x) in _dispatch._PLAIN_TENSOR_TYPES and x.dtype in dtypes
            for x in t if isinstance(x, torch.Tensor)))


@pytest.fixture
def contest(monkeypatch, tmp_path):
    """kernel_select on, timing stubbed by candidate name, disk cache off."""
    monkeypatch.setattr(kernel_select, "_ENABLED", True)
    monkeypatch.setattr(kernel_select, "_DISK_CACHE_ENABLED", False)
    table = {}

    def fake_time(fn):  # candidate thunks are tagged with their name by _tag()
        if fn() is None:
            return None
        return table.get(getattr(fn, "_n", ""), 1.0)
    monkeypatch.setattr(kernel_select, "_time", fake_time)
    kernel_select.reset()
    yield table
    kernel_select.reset()


def _tag(cands):
    for n, t in cands:
        t._n = n
    return cands


def test_conv3d_contest_over_native_variants_then_cached(monkeypatch, contest):
    fake = FakeNative(monkeypatch, ["h_a", "h_b", "f32_c"], ["res", "twopass"])
    monkeypatch.setattr(_dispatch, "_conv_candidates",
                        (lambda orig: (lambda *a: _tag(orig(*a))))(_dispatch._conv_candidates))
    contest.update({"native.h_a": 3.0, "native.h_b": 1.0, "stock": 2.0})
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, 4, 4, 5, 6, generator=g).half()
    w = torch.randn(4, 4, 3, 3, 3, generator=g).half()
    with torch.no_grad():
        y = F.conv3d(x.float(), w.float(), None, 1, 1).half()  # fp32 path: only f32_ variants
    fake.calls.clear()
    kernel_select.reset()
    x32, w32 = x.float(), w.float()
    contest.update({"native.f32_c": 0.5})
    out = F.conv3d(x32, w32, None, 1, 1)
    assert kernel_select.cached("conv3d", x32, w32, 1, 1, 1) == "native.f32_c"
    assert ("conv3d", "h_a") not in fake.calls      # 16-bit variants never offered for fp32
    fake.calls.clear()
    F.conv3d(x32, w32, None, 1, 1)
    assert fake.calls == [("conv3d", "f32_c")]       # cached: straight to the winner
    assert torch.allclose(out, y.float(), atol=1e-2, rtol=2e-3)  # y went through fp16 rounding


def test_conv3d_cached_winner_declining_is_recontested(monkeypatch, contest):
    fake = FakeNative(monkeypatch, ["f32_a", "f32_b"], ["res"])
    monkeypatch.setattr(_dispatch, "_conv_candidates",
                        (lambda orig: (lambda *a: _tag(orig(*a))))(_dispatch._conv_candidates))
    contest.update({"native.f32_a": 0.5, "native.f32_b": 1.0, "stock": 2.0})
    x, w = torch.randn(1, 2, 3, 4, 5), torch.randn(3, 2, 3, 3, 3)
    F.conv3d(x, w, None, 1, 1)
    assert kernel_select.cached("conv3d", x, w, 1, 1, 1) == "native.f32_a"
    fake.decline.add("f32_a")
    F.conv3d(x, w, None, 1, 1)
    assert kernel_select.cached("conv3d", x, w, 1, 1, 1) == "native.f32_b"


def test_conv_gates_send_to_stock(monkeypatch, contest):
    fake = FakeNative(monkeypatch, ["f32_a"], ["res"])
    x, w = torch.randn(1, 4, 6, 6), torch.randn(4, 1, 3, 3)
    F.conv2d(x, w, None, 1, 1, 1, 4)                               # grouped
    F.conv2d(x, torch.randn(4, 4, 1, 1))                           # pointwise 1x1
    F.conv2d(x.transpose(2, 3), torch.randn(4, 4, 3, 3), None, 1, 1)  # neither contiguous nor channels-last
    F.conv2d(x, torch.randn(4, 4, 3, 3), None, 1, "same")          # string padding
    F.conv2d(x.double(), torch.randn(4, 4, 3, 3).double())         # dtype outside the tier
    assert fake.calls == []


def test_conv_channels_last_contests_native_on_nchw_copies(monkeypatch, contest):
    """Channels-last input and weight enter the contest: the native candidates run on NCHW
    copies, hand the output back channels-last like stock, and the winner is keyed on the
    memory format."""
    fake = FakeNative(monkeypatch, ["f32_a"], ["res"])
    seen = []
    orig_conv2d = _native.conv2d

    def spy(input, weight, *a, **k):
        seen.append((input.is_contiguous(), weight.is_contiguous()))
        return orig_conv2d(input, weight, *a, **k)
    monkeypatch.setattr(_native, "conv2d", spy)
    contest.update({"native.f32_a": 0.5, "stock": 2.0})
    x = torch.randn(1, 4, 6, 6).to(memory_format=torch.channels_last)
    w = torch.randn(5, 4, 3, 3).to(memory_format=torch.channels_last)
    y = F.conv2d(x, w, None, 1, 1)
    assert set(fake.calls) == {("conv2d", "f32_a"), ("layout", "to_ncdhw"), ("layout", "to_channels_last")}
    assert seen and set(seen) == {(True, True)}
    assert y.is_contiguous(memory_format=torch.channels_last)
    assert torch.allclose(y, _dispatch._ORIGINALS[(F, "conv2d")](x, w, None, 1, 1), atol=1e-5)
    assert kernel_select.cached("conv2d", x, w, 1, 1, 1) == "native.f32_a"
    assert kernel_select.cached("conv2d", x.contiguous(), w, 1, 1, 1) is None  # layout in the key


def test_conv_channels_last_16bit_takes_the_channels_last_tiles(monkeypatch, contest):
    """A 16-bit channels-last input goes to the tiles that stage channels-last patches
    (no layout conversions); where they decline, the NC(D)HW copies are used."""
    fake = FakeNative(monkeypatch, ["h_a", "h_b"], ["res"])
    cl_calls = []

    def conv_cl(input, weight, bias, stride, padding, dilation, nd, *, variant):
        cl_calls.append(variant)
        if variant == 2:
            raise _native.Unsupported("declined")
        ref = _dispatch._ORIGINALS[(F, "conv%dd" % nd)](input.float(), weight.float(),
                                                       None if bias is None else bias.float(),
                                                       stride, padding, dilation)
        return ref.to(input.dtype).contiguous(memory_format=torch.channels_last)
    monkeypatch.setattr(_native, "conv_channels_last", conv_cl)
    contest.update({"native.h_a": 0.5, "native.h_b": 0.4, "stock": 2.0})
    x = torch.randn(1, 8, 6, 6).to(torch.bfloat16).to(memory_format=torch.channels_last)
    w = torch.randn(8, 8, 3, 3).to(torch.bfloat16)
    y = F.conv2d(x, w, None, 1, 1)
    assert set(cl_calls) == {1, 2}                           # both candidates tried the tiles
    assert ("conv2d", "h_a") not in fake.calls               # h_a ran channels-last, no copy
    assert ("conv2d", "h_b") in fake.calls                   # h_b declined: NCHW copies
    assert y.is_contiguous(memory_format=torch.channels_last)


def test_group_norm_contest_and_key(monkeypatch, contest):
    fake = FakeNative(monkeypatch, ["f32_a"], ["res_a", "twopass"])
    monkeypatch.setattr(_dispatch, "_group_norm_candidates",
                        (lambda orig: (lambda *a, **k: _tag(orig(*a, **k))))(_dispatch._group_norm_candidates))
    contest.update({"native.res_a": 0.3, "native.twopass": 0.6, "stock": 1.0})
    x = torch.randn(2, 8, 4, 4)
    y = F.group_norm(x, 4, torch.ones(8), torch.zeros(8), 1e-5)
    key = (x.dtype, tuple(x.shape), 4, False)
    assert kernel_select.cached_key("group_norm", key) == "native.res_a"
    fake.calls.clear()
    y2 = F.group_norm(x, 4, torch.ones(8), torch.zeros(8), 1e-5)
    assert fake.calls == [("group_norm", "res_a")]
    assert torch.equal(y, y2)
    # non-contiguous input never reaches the native layer
    fake.calls.clear()
    F.group_norm(x.transpose(2, 3), 4)
    assert fake.calls == []


def test_kernel_select_off_uses_fixed_native_order(monkeypatch):
    monkeypatch.setattr(kernel_select, "_ENABLED", False)
    fake = FakeNative(monkeypatch, ["f32_a", "f32_b"], ["res_a", "twopass"], decline={"res_a", "f32_a"})
    x = torch.randn(2, 8, 4, 4)
    F.group_norm(x, 4)
    assert fake.calls == [("group_norm", "res_a"), ("group_norm", "twopass")]
    fake.calls.clear()
    F.conv2d(x, torch.randn(3, 8, 3, 3), None, 1, 1)
    assert fake.calls == [("conv2d", "f32_a"), ("conv2d", "f32_b")]


def test_sequential_groupnorm_silu_conv_fusion(monkeypatch):
    calls = []
    monkeypatch.setattr(conv_fusion_ops, "group_norm_silu",
                        lambda x, G, w, b, eps: calls.append(G) or F.silu(
                            _dispatch._ORIGINALS[(F, "group_norm")](x, G, w, b, eps)))
    installed = (nn.Sequential, "forward") in _dispatch._ORIGINALS
    if not installed:
        monkeypatch.setattr(_dispatch, "_SEQ_FORWARD_ORIG", nn.Sequential.forward)
    fwd = _dispatch._patched_sequential_forward
    seq = nn.Sequential(nn.GroupNorm(2, 4), nn.SiLU(), nn.Conv2d(4, 3, 3, padding=1))
    x = torch.randn(1, 4, 6, 6)
    with torch.no_grad():
        ref = seq[2](F.silu(seq[0](x)))
        out = fwd(seq, x)
    assert calls == [2] and torch.allclose(out, ref, atol=1e-6)
    other = nn.Sequential(nn.GroupNorm(2, 4), nn.ReLU(), nn.Conv2d(4, 3, 3, padding=1))
    calls.clear()
    with torch.no_grad():
        fwd(other, x)
    assert calls == []


def test_sequential_conv_groupnorm_silu_fusion(monkeypatch):
    """The conv-first (video VAE decoder) order: Conv3d, GroupNorm(affine), SiLU."""
    calls = []
    monkeypatch.setattr(conv_fusion_ops, "group_norm_silu",
                        lambda x, G, w, b, eps: calls.append(G) or F.silu(
                            _dispatch._ORIGINALS[(F, "group_norm")](x, G, w, b, eps)))
    if (nn.Sequential, "forward") not in _dispatch._ORIGINALS:
        monkeypatch.setattr(_dispatch, "_SEQ_FORWARD_ORIG", nn.Sequential.forward)
    fwd = _dispatch._patched_sequential_forward
    seq = nn.Sequential(nn.Conv3d(4, 4, 3, padding=1), nn.GroupNorm(2, 4, eps=1e-6), nn.SiLU())
    x = torch.randn(1, 4, 3, 5, 5)
    with torch.no_grad():
        ref = F.silu(seq[1](seq[0](x)))
        out = fwd(seq, x)
    assert calls == [2] and torch.allclose(out, ref, atol=1e-6)
    calls.clear()
    with torch.no_grad():
        fwd(nn.Sequential(nn.Conv3d(4, 4, 3, padding=1), nn.GroupNorm(2, 4), nn.ReLU()), x)
        fwd(nn.Sequential(nn.Conv3d(4, 4, 3, padding=1), nn.GroupNorm(2, 4, affine=False), nn.SiLU()), x)
    assert calls == []


def test_replace_and_unfuse_vae_blocks(monkeypatch):
    monkeypatch.setattr(conv_fusion_ops, "enabled", lambda: True)
    model = nn.Sequential(nn.Sequential(nn.Conv3d(4, 4, 3, padding=1), nn.GroupNorm(2, 4), nn.SiLU()),
                          nn.Sequential(nn.Conv2d(4, 4, 3, padding=1), nn.GroupNorm(2, 4), nn.SiLU()))
    keys = set(model.state_dict().keys())
    conv3 = model[0][0]
    assert conv_fusion_ops.replace_conv_blocks(model) == 2
    assert isinstance(model[0], conv_fusion_ops.FusedConvGroupNormSiLU)
    assert model[0].conv is conv3 and set(model.state_dict().keys()) == keys
    assert conv_fusion_ops.replace_conv_blocks(model) == 0
    x = torch.randn(1, 4, 3, 5, 5)
    with torch.no_grad():
        fused = model[0](x)
    assert conv_fusion_ops.unfuse_conv_blocks(model) == 2
    with torch.no_grad():
        assert torch.allclose(model[0](x), fused, atol=1e-6)


def test_replace_and_unfuse_conv_blocks(monkeypatch):
    monkeypatch.setattr(conv_fusion_ops, "enabled", lambda: True)
    model = nn.Sequential(nn.Sequential(nn.GroupNorm(2, 4), nn.SiLU(), nn.Conv2d(4, 4, 3, padding=1)),
                          nn.Sequential(nn.GroupNorm(2, 4), nn.ReLU(), nn.Conv2d(4, 4, 3, padding=1)))
    keys = set(model.state_dict().keys())
    gn = model[0][0]
    assert conv_fusion_ops.replace_conv_blocks(model) == 1
    assert isinstance(model[0], conv_fusion_ops.FusedGroupNormSiLUConv2d)
    assert model[0].norm is gn and set(model.state_dict().keys()) == keys
    assert conv_fusion_ops.replace_conv_blocks(model) == 0          # idempotent
    x = torch.randn(1, 4, 5, 5)
    with torch.no_grad():
        fused = model(x)
    assert conv_fusion_ops.unfuse_conv_blocks(model) == 1
    with torch.no_grad():
        assert torch.allclose(model(x), fused, atol=1e-6)


def test_dispatch_debug_counters(monkeypatch):
    monkeypatch.setattr(_dispatch, "_DEBUG", True)
    _dispatch.dispatch_debug_reset()
    F.conv2d(torch.randn(1, 4, 6, 6), torch.randn(4, 1, 3, 3), None, 1, 1, 1, 4)
    counts = _dispatch.dispatch_debug_counts()
    assert counts.get(("conv2d", "stock")) == 1
    assert "conv2d" in _dispatch.dispatch_debug_report()
    _dispatch.dispatch_debug_reset()
    assert "no routing decisions" in _dispatch.dispatch_debug_report()


def test_torchscript_guard_compiles_against_stock():
    def f(x, w):
        return F.conv2d(x, w, None, 1, 1)
    scripted = torch.jit.script(f)
    assert att.is_enabled()
    x, w = torch.randn(1, 2, 5, 5), torch.randn(3, 2, 3, 3)
    assert torch.allclose(scripted(x, w), _dispatch._ORIGINALS[(F, "conv2d")](x, w, None, 1, 1))
    traced = torch.jit.trace(lambda x: F.group_norm(x, 2), (torch.randn(1, 4, 3, 3),))
    assert att.is_enabled()
    t = torch.randn(1, 4, 3, 3)
    assert torch.allclose(traced(t), torch.group_norm(t, 2))


# ---------------------------------------------------------------------------
# autograd wrappers (backward = stock math), checked in float64
# ---------------------------------------------------------------------------
def test_group_norm_backward_matches_autograd_fp64():
    torch.manual_seed(0)
    for affine in (True, False):
        x = torch.randn(3, 8, 5, 4, dtype=torch.float64, requires_grad=True)
        w = torch.randn(8, dtype=torch.float64, requires_grad=True) if affine else None
        b = torch.randn(8, dtype=torch.float64, requires_grad=True) if affine else None
        y = torch.group_norm(x, 4, w, b, 1e-5)
        dy = torch.randn_like(y)
        refs = torch.autograd.grad(y, [t for t in (x, w, b) if t is not None], dy)
        gx, gw, gb = _dispatch._group_norm_backward(dy, x.detach(), 4, None if w is None else w.detach(),
                                                    1e-5, (True, affine, affine))
        torch.testing.assert_close(gx, refs[0], rtol=1e-10, atol=1e-10)
        if affine:
            torch.testing.assert_close(gw, refs[1], rtol=1e-10, atol=1e-10)
            torch.testing.assert_close(gb, refs[2], rtol=1e-10, atol=1e-10)


def test_conv_autograd_wrapper_backward(monkeypatch):
    """_ConvFn: forward through the given function, backward through
    aten.convolution_backward -- equal to stock's gradients."""
    torch.manual_seed(1)
    x = torch.randn(1, 2, 4, 5, 6, dtype=torch.float64, requires_grad=True)
    w = torch.randn(3, 2, 3, 3, 3, dtype=torch.float64, requires_grad=True)
    b = torch.randn(3, dtype=torch.float64, requires_grad=True)
    orig = _dispatch._ORIGINALS[(F, "conv3d")]
    y = _dispatch._ConvFn.apply(x, w, b, 1, 1, 1, 1, 3, lambda *a: orig(*a))
    dy = torch.randn_like(y)
    g = torch.autograd.grad(y, (x, w, b), dy)
    y2 = orig(x, w, b, 1, 1, 1, 1)
    g2 = torch.autograd.grad(y2, (x, w, b), dy)
    for a, r in zip(g, g2):
        torch.testing.assert_close(a, r)


def test_dwconv1d_autograd_backward_matches_stock(monkeypatch):
    """The depthwise conv1d autograd wrapper's backward (stock convolution_backward on the
    left/right padded input) equals autograd through stock F.conv1d, for the symmetric,
    causal stock-shape and truncated-causal forms."""
    torch.manual_seed(2)

    def fake_dw(x, w, b, pad_left, l_out, silu=False, variant=-1, out=None):
        xp = F.pad(x, (pad_left, max(0, l_out + w.shape[1] - 1 - x.shape[-1] - pad_left)))
        return STOCK_CONV1D(xp, w.unsqueeze(1), b, 1, 0, 1, x.shape[1])[..., :l_out]
    monkeypatch.setattr(_native, "dwconv1d", fake_dw)
    for K, pad, l_out in ((3, 1, 10), (4, 3, 13), (4, 3, 10)):
        x = torch.randn(2, 3, 10, dtype=torch.float64, requires_grad=True)
        w = torch.randn(3, 1, K, dtype=torch.float64, requires_grad=True)
        b = torch.randn(3, dtype=torch.float64, requires_grad=True)
        y = miopen_fallback._DwConv1dFn.apply(x, w, b, pad, l_out, -1)
        ref = STOCK_CONV1D(x, w, b, 1, pad, 1, 3)[..., :l_out]
        torch.testing.assert_close(y, ref)
        dy = torch.randn_like(y)
        for a, r in zip(torch.autograd.grad(y, (x, w, b), dy), torch.autograd.grad(ref, (x, w, b), dy)):
            torch.testing.assert_close(a, r)


def test_conv1d_padding_resolution():
    assert miopen_fallback._resolve_padding(1, 3, 10) == (1, 10)
    assert miopen_fallback._resolve_padding((3,), 4, 10) == (3, 13)
    assert miopen_fallback._resolve_padding("valid", 5, 10) == (0, 6)
    assert miopen_fallback._resolve_padding("same", 4, 10) == (1, 10)
    assert miopen_fallback._resolve_padding(65, 3, 10) is None
    assert miopen_fallback._resolve_padding("circular", 3, 10) is None


def test_conv_dgrad_as_forward_conv_matches_stock():
    """The input gradient of a stride-1 conv equals the forward conv of dy with the weights
    swapped in (Co, Ci) and flipped in space, padding k-1-p -- the identity _ConvFn's
    backward uses on the GPU -- for conv3d and conv2d, asymmetric kernels and paddings."""
    torch.manual_seed(4)
    for nd, xs, ws, pad in ((3, (2, 3, 5, 6, 7), (4, 3, 3, 2, 3), (1, 0, 2)),
                            (2, (1, 2, 7, 6), (3, 2, 3, 3), (1, 1)),
                            (3, (1, 2, 6, 6, 6), (2, 2, 3, 3, 3), (0, 0, 0))):
        x = torch.randn(*xs, dtype=torch.float64, requires_grad=True)
        w = torch.randn(*ws, dtype=torch.float64)
        conv = torch.nn.functional.conv3d if nd == 3 else torch.nn.functional.conv2d
        stock = _dispatch._ORIGINALS[(torch.nn.functional, "conv3d" if nd == 3 else "conv2d")]
        y = stock(x, w, None, 1, pad, 1, 1)
        dy = torch.randn_like(y)
        ref, = torch.autograd.grad(y, x, dy)
        pad_t = _dispatch._dgrad_padding(w, 1, pad, 1, 1, nd)
        got = _dispatch._dgrad_via_forward(dy, w, pad_t, nd, lambda i, ww, b, s, p, d, g: stock(i, ww, b, s, p, d, g))
        torch.testing.assert_close(got, ref)
        del conv
    w = torch.zeros(2, 2, 3, 3, 3)
    assert _dispatch._dgrad_padding(w, 2, 1, 1, 1, 3) is None          # stride 2
    assert _dispatch._dgrad_padding(w, 1, 1, 2, 1, 3) is None          # dilation 2
    assert _dispatch._dgrad_padding(w, 1, 3, 1, 1, 3) is None          # padding > k-1
    assert _dispatch._dgrad_padding(w, 1, "same", 1, 1, 3) is None


# ---------------------------------------------------------------------------
# MIOpen rescue and the reference-shape causal mode (reference tests/test_miopen_fallback.py,
# miopen_fallback.py:450-483)
# ---------------------------------------------------------------------------
def _conv1d_args(dtype=torch.float16):
    g = torch.Generator().manual_seed(7)
    x = torch.randn(2, 4, 16, generator=g).to(dtype)
    w = torch.randn(6, 4, 3, generator=g).to(dtype)
    b = torch.randn(6, generator=g).to(dtype)
    return x, w, b


def test_miopen_failure_is_rescued_on_cpu_in_fp32(capsys):
    """An `orig` raising a miopenStatus error: the conv runs on the CPU in fp32 and comes back
    in the input's dtype (a CPU input has no GPU retry), with the reference's notice."""
    x, w, b = _conv1d_args()
    calls = []

    def flaky(inp, wt, bs, stride, padding, dilation, groups):
        calls.append(inp.dtype)
        if inp.dtype != torch.float32:
            raise RuntimeError("miopenStatusUnknownError: conv failed")
        return STOCK_CONV1D(inp, wt, bs, stride, padding, dilation, groups)

    wrapped = miopen_fallback._miopen_safe_conv("conv1d", flaky)
    y = wrapped(x, w, b, 1, 1)
    ref = STOCK_CONV1D(x.float(), w.float(), b.float(), 1, 1).to(torch.float16)
    assert y.dtype == torch.float16 and torch.equal(y, ref)
    assert calls == [torch.float16, torch.float32]
    assert "MIOpen fallback (conv1d): CPU used" in capsys.readouterr().out


def test_miopen_rescue_leaves_other_errors_alone():
    x, w, b = _conv1d_args()

    def broken(*a):
        raise RuntimeError("shape mismatch")
    with pytest.raises(RuntimeError, match="shape mismatch"):
        miopen_fallback._miopen_safe_conv("conv1d", broken)(x, w, b, 1, 1)


def test_miopen_rescue_retries_gpu_call_after_empty_cache(monkeypatch):
    """A GPU input is tried twice (the second time after torch.cuda.empty_cache()) before
    the CPU fallback; a retry that succeeds is returned as is."""
    x, w, b = _conv1d_args()

    class GpuLike:  # stands in for a tensor that reports is_cuda (no GPU here)
        is_cuda = True
        shape = x.shape

    attempts, emptied = [], []
    monkeypatch.setattr(torch.cuda, "empty_cache", lambda: emptied.append(len(attempts)))

    def once_flaky(inp, *rest):
        attempts.append(1)
        if len(attempts) == 1:
            raise RuntimeError("miopenStatusInternalError")
        return "second try"
    out = miopen_fallback._stock_with_rescue("conv1d", once_flaky, GpuLike(), w, b, 1, 1, 1, 1)
    assert out == "second try" and len(attempts) == 2 and emptied == [1]


def test_causal_truncate_mode_gate(monkeypatch):
    """AMD_TUNED_TORCH_CAUSAL_CONV1D_TRUNCATE=1 turns on the length-L causal path; it stays
    off by default and never serves CPU tensors."""
    x = torch.randn(2, 4, 32)
    w = torch.randn(4, 1, 4)
    monkeypatch.setattr(miopen_fallback, "_CAUSAL_TRUNCATE", False)
    assert miopen_fallback._try_causal_conv1d_fastpath(x, w, None, 1, 3, 1, 4) is None
    monkeypatch.setattr(miopen_fallback, "_CAUSAL_TRUNCATE", True)
    assert miopen_fallback._try_causal_conv1d_fastpath(x, w, None, 1, 3, 1, 4) is None  # CPU
    assert miopen_fallback._is_causal_conv1d_eligible(x, w, 1, 3, 1, 4) is False       # not cuda
    y = F.conv1d(x, w, None, 1, 3, 1, 4)  # CPU: stock shape either way
    assert y.shape == (2, 4, 35)


def test_workspaces_are_private_per_stream_and_retired_on_growth(monkeypatch):
    """Scratch is pooled per (device, stream, purpose); a grown buffer replaces the old one,
    which stays alive (a captured graph may still point at it)."""
    current = [11]
    monkeypatch.setattr(_native, "_raw_stream", lambda device: current[0])
    real_zeros = torch.zeros
    monkeypatch.setattr(torch, "zeros", lambda n, dtype=None, device=None: real_zeros(n, dtype=dtype))
    monkeypatch.setattr(_native, "_ws_live", {})
    monkeypatch.setattr(_native, "_ws_retired", [])
    dev = torch.device("cuda", 0)
    a = _native.workspace(dev, "conv", 100)
    assert _native.workspace(dev, "conv", 50) is a            # same stream, fits: reused
    current[0] = 22
    b = _native.workspace(dev, "conv", 100)
    assert b is not a                                         # another stream: its own buffer
    current[0] = 11
    grown = _native.workspace(dev, "conv", 1 << 20)
    assert grown.numel() >= 1 << 20 and grown is not a
    assert any(r is a for r in _native._ws_retired)           # retired, not freed
    assert _native.workspace_keys() == [(0, 11, "conv"), (0, 22, "conv")]
