"""GPU parity of the dense conv2d/conv3d kernels (C ABI atk_conv_fwd), every variant,
against the float64 oracle.  Bars: fp32 <= 1e-5 max-abs-rel, fp16/bf16 <= 1e-2."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
BAR = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 1e-2}


def _native():
    from amd_tuned_torch import _native
    return _native


def _inputs(xshape, wshape, dtype, seed=0, bias=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*xshape, generator=g)
    fan_in = math.prod(wshape[1:])
    w = torch.randn(*wshape, generator=g) * math.sqrt(2.0 / fan_in)  # kaiming-normal
    b = torch.randn(wshape[0], generator=g) * 0.1 if bias else None
    return x.to(dtype), w.to(dtype), (b.to(dtype) if bias else None)


def _variants_for(dtype):
    nat = _native()
    names = nat.variants(nat.OP_CONV)
    out = []
    for i, n in enumerate(names):
        if n.startswith("f32_") and dtype != torch.float32:
            continue
        if n.startswith("h_") and dtype == torch.float32:
            continue
        out.append((i, n))
    return out


CONV3D = [
    # xshape, wshape, stride, padding, dilation
    ((1, 8, 6, 7, 9), (16, 8, 3, 3, 3), 1, 1, 1),
    ((2, 5, 5, 6, 7), (3, 5, 3, 3, 3), 1, 1, 1),           # channel counts off the tiles
    ((1, 16, 4, 9, 10), (8, 16, 1, 3, 3), (1, 2, 2), (0, 1, 1), 1),
    ((1, 4, 7, 8, 9), (6, 4, 3, 2, 3), (2, 1, 1), (1, 0, 2), (1, 2, 1)),
    ((1, 32, 8, 16, 16), (64, 32, 3, 3, 3), 1, 1, 1),
    ((1, 8, 9, 9, 9), (8, 8, 5, 5, 5), 1, 2, 1),
    # stage counts that the in-workgroup K split divides unevenly (some K groups idle)
    ((1, 40, 5, 12, 16), (32, 40, 3, 3, 3), 1, 1, 1),
    ((1, 16, 6, 16, 16), (16, 16, 7, 7, 7), 1, 3, 1),
]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("case", CONV3D, ids=lambda c: "x".join(map(str, c[0])) + "_w" + "x".join(map(str, c[1])))
def test_conv3d_all_variants(dev, case, dtype):
    xs, ws, s, p, d = case
    nat = _native()
    x, w, b = _inputs(xs, ws, dtype, seed=sum(xs))
    ref = O.conv3d(x, w, b, s, p, d)
    for vi, name in _variants_for(dtype):
        try:
            y = nat.conv3d(x.to(dev), w.to(dev), b.to(dev), s, p, d, variant=vi)
        except nat.Unsupported:
            continue
        torch.cuda.synchronize()
        assert tuple(y.shape) == ref.shape
        err = O.max_rel_err(y.cpu(), ref)
        assert err <= BAR[dtype], f"{name}: max_rel_err {err:.3g}"


CONV2D = [
    ((2, 8, 13, 17), (16, 8, 3, 3), 1, 1, 1),
    ((1, 16, 20, 20), (8, 16, 3, 3), 2, 1, 1),
    ((1, 3, 11, 12), (5, 3, 5, 3), 1, (2, 1), (1, 2)),
]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("case", CONV2D, ids=lambda c: "x".join(map(str, c[0])))
def test_conv2d_all_variants(dev, case, dtype):
    xs, ws, s, p, d = case
    nat = _native()
    x, w, b = _inputs(xs, ws, dtype, seed=sum(xs))
    ref = O.conv2d(x, w, b, s, p, d)
    for vi, name in _variants_for(dtype):
        try:
            y = nat.conv2d(x.to(dev), w.to(dev), b.to(dev), s, p, d, variant=vi)
        except nat.Unsupported:
            continue
        torch.cuda.synchronize()
        err = O.max_rel_err(y.cpu(), ref)
        assert err <= BAR[dtype], f"{name}: max_rel_err {err:.3g}"


def test_conv_no_bias(dev):
    nat = _native()
    x, w, _ = _inputs((1, 8, 4, 6, 6), (8, 8, 3, 3, 3), torch.float32, seed=4, bias=False)
    ref = O.conv3d(x, w, None, 1, 1, 1)
    for vi, name in _variants_for(torch.float32):
        try:
            y = nat.conv3d(x.to(dev), w.to(dev), None, 1, 1, 1, variant=vi)
        except nat.Unsupported:
            continue
        torch.cuda.synchronize()
        assert O.max_rel_err(y.cpu(), ref) <= 1e-5, name


CONFIGS = [
    # BASELINE configs 4 and 5: (xshape, wshape, padding, dtype)
    ((1, 64, 16, 32, 32), (64, 64, 3, 3, 3), 1, torch.float16),
    ((1, 64, 16, 32, 32), (64, 64, 3, 3, 3), 1, torch.float32),
    ((2, 128, 16, 64, 64), (128, 128, 3, 3, 3), 1, torch.bfloat16),
    ((1, 256, 8, 64, 64), (256, 256, 3, 3, 3), 1, torch.bfloat16),
    ((1, 64, 16, 32, 32), (64, 64, 7, 7, 7), 3, torch.float16),
]


@pytest.mark.parametrize("cfg", CONFIGS, ids=["c4_small_fp16", "c4_small_fp32", "c4_scaled_bf16",
                                               "c5_bf16", "c5_k7_fp16"])
def test_conv3d_config_full_size(dev, cfg):
    """Every MFMA variant at the BASELINE shapes: 4096 sampled outputs against the float64
    oracle, and every output against stock F.conv3d in fp32 on the same inputs."""
    xs, ws, pad, dtype = cfg
    nat = _native()
    x, w, b = _inputs(xs, ws, dtype, seed=1004)
    g = torch.Generator().manual_seed(7)
    oshape = O.conv_out_shape(xs, ws, 1, pad, 1)
    pts = torch.randint(0, math.prod(oshape), (4096,), generator=g).numpy()
    ref_pts = O.conv3d(x, w, b, 1, pad, 1, points=pts)
    xd, wd, bd = x.to(dev), w.to(dev), b.to(dev)
    stock = torch.nn.functional.conv3d  # the package may be imported: use aten directly
    ref_full = torch.ops.aten.convolution(xd.float(), wd.float(), bd.float(), [1, 1, 1], [pad] * 3,
                                          [1, 1, 1], False, [0, 0, 0], 1)
    ran = 0
    for vi, name in _variants_for(dtype):
        if name == "direct":
            continue
        try:
            y = nat.conv3d(xd, wd, bd, 1, pad, 1, variant=vi)
        except nat.Unsupported:
            continue
        torch.cuda.synchronize()
        yp = y.flatten()[torch.from_numpy(pts).to(dev)].cpu()
        e1 = float(np.max(np.abs(O.f64(yp) - ref_pts)) / np.max(np.abs(ref_pts)))
        e2 = O.max_rel_err(y.float(), ref_full)
        assert e1 <= BAR[dtype], f"{name}: sampled max_rel_err {e1:.3g}"
        assert e2 <= max(BAR[dtype], 2e-5 if dtype == torch.float32 else 0), f"{name}: vs stock {e2:.3g}"
        ran += 1
    del stock
    assert ran >= 1


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_conv3d_autograd_dgrad_through_forward(dev, dtype):
    """Training path: patched F.conv3d with requires_grad runs the accelerated forward, the
    input gradient through the same forward on dy with transposed / flipped weights, and
    the weight / bias gradients through aten -- all equal to float64 autograd on the CPU."""
    import torch.nn.functional as F
    import amd_tuned_torch  # noqa: F401
    g = torch.Generator().manual_seed(12)
    x = torch.randn(2, 32, 6, 16, 16, generator=g)
    w = torch.randn(48, 32, 3, 3, 3, generator=g) * 0.05
    b = torch.randn(48, generator=g) * 0.1
    xd = x.to(dtype).to(dev).requires_grad_(True)
    wd = w.to(dtype).to(dev).requires_grad_(True)
    bd = b.to(dtype).to(dev).requires_grad_(True)
    y = F.conv3d(xd, wd, bd, 1, 1)
    dy = torch.randn(y.shape, generator=g)
    gx, gw, gb = torch.autograd.grad(y, (xd, wd, bd), dy.to(dtype).to(dev))
    x64, w64, b64 = (t.to(dtype).double().requires_grad_(True) for t in (x, w, b))
    y64 = torch.nn.functional.conv3d(x64, w64, b64, 1, 1)
    rx, rw, rb = torch.autograd.grad(y64, (x64, w64, b64), dy.to(dtype).double())
    bar = 1e-5 if dtype == torch.float32 else 1e-2
    for got, ref in ((gx, rx), (gw, rw), (gb, rb)):
        err = (got.double().cpu() - ref).abs().max().item() / ref.abs().max().item()
        assert err <= bar, err


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_vae_block_fused_forward_and_grads(dtype):
    """Config 5's block order, Conv3d(C->C, k3, pad 1) -> GroupNorm(32, eps 1e-6) -> SiLU, at a
    reduced size: replace_conv_blocks fuses it (accelerated conv, fused GroupNorm+SiLU);
    the output and, with gradients live, the parameter and input gradients match a float64
    CPU run of the unfused stock block."""
    import torch.nn as nn
    import amd_tuned_torch
    from amd_tuned_torch import conv_fusion_ops
    torch.manual_seed(0)
    C = 64
    block = nn.Sequential(nn.Conv3d(C, C, 3, padding=1), nn.GroupNorm(32, C, eps=1e-6), nn.SiLU())
    with torch.no_grad():
        block[1].weight.normal_(1.0, 0.1)
        block[1].bias.normal_(0.0, 0.1)
    import copy
    ref_block = copy.deepcopy(block).double()
    model = nn.Sequential(copy.deepcopy(block)).to("cuda", dtype)
    assert conv_fusion_ops.replace_conv_blocks(model) == 1
    assert isinstance(model[0], conv_fusion_ops.FusedConvGroupNormSiLU)
    x = torch.randn(1, C, 4, 16, 16)
    bar = 1e-2 if dtype == torch.bfloat16 else 1e-5
    with torch.no_grad():
        y = model(x.to("cuda", dtype))
        amd_tuned_torch.disable()
        try:
            ref = ref_block(x.double())
        finally:
            amd_tuned_torch.enable()
    assert O.max_rel_err(y.float(), ref) <= bar
    # training: gradients through the accelerated conv (dgrad on the forward kernels) and the
    # native GroupNorm backward
    xg = x.to("cuda", dtype).requires_grad_()
    out = model(xg)
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(1))
    out.backward(g.to("cuda", dtype))
    xr = x.double().requires_grad_()
    amd_tuned_torch.disable()
    try:
        ref_block(xr).backward(g.double())
    finally:
        amd_tuned_torch.enable()
    assert O.max_rel_err(xg.grad.float(), xr.grad) <= bar
    fused = model[0]
    for got, want in ((fused.conv.weight.grad, ref_block[0].weight.grad), (fused.conv.bias.grad, ref_block[0].bias.grad),
                      (fused.norm.weight.grad, ref_block[1].weight.grad), (fused.norm.bias.grad, ref_block[1].bias.grad)):
        assert O.max_rel_err(got.float(), want) <= bar


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("nd", [2, 3])
def test_channels_last_conv_through_patched_functional(nd, dtype):
    """Channels-last (NHWC / NDHWC) input and weight through patched F.conv2d / F.conv3d:
    the contest includes the native tiles (on NC(D)HW copies) and returns the output in the
    input's channels-last layout, like stock; values match the float64 oracle."""
    import torch.nn.functional as F
    import amd_tuned_torch
    from amd_tuned_torch import kernel_select
    g = torch.Generator().manual_seed(nd)
    if nd == 3:
        x = torch.randn(1, 32, 6, 20, 20, generator=g)
        w = torch.randn(48, 32, 3, 3, 3, generator=g) / math.sqrt(32 * 27)
        fmt, conv = torch.channels_last_3d, F.conv3d
    else:
        x = torch.randn(2, 32, 24, 24, generator=g)
        w = torch.randn(48, 32, 3, 3, generator=g) / math.sqrt(32 * 9)
        fmt, conv = torch.channels_last, F.conv2d
    b = torch.randn(48, generator=g) * 0.1
    xd = x.to("cuda", dtype).contiguous(memory_format=fmt)
    wd = w.to("cuda", dtype).contiguous(memory_format=fmt)
    bd = b.to("cuda", dtype)
    assert amd_tuned_torch.is_enabled()
    y = conv(xd, wd, bd, 1, 1)
    assert y.is_contiguous(memory_format=fmt)
    won = kernel_select.cached("conv3d" if nd == 3 else "conv2d", xd, wd, 1, 1, 1)
    assert won is not None
    ref = (O.conv3d if nd == 3 else O.conv2d)(x.to(dtype), w.to(dtype), b.to(dtype), 1, 1, 1)
    bar = 1e-5 if dtype == torch.float32 else 1e-2
    assert O.max_rel_err(y.float().contiguous(), ref) <= bar, won
    y2 = conv(xd, wd, bd, 1, 1)  # cached-winner path
    assert y2.is_contiguous(memory_format=fmt) and O.max_rel_err(y2.float().contiguous(), ref) <= bar


CL_NATIVE_CASES = [
    # xshape (logical NC[D]HW), wshape, padding: 3x3(x3) and 7x7x7 planes, edges, odd sizes
    ((1, 32, 6, 20, 20), (48, 32, 3, 3, 3), 1),
    ((2, 64, 4, 9, 13), (32, 64, 3, 3, 3), 1),
    ((1, 16, 5, 12, 12), (16, 16, 7, 7, 7), 3),
    ((2, 40, 17, 11), (24, 40, 3, 3), 1),
    ((1, 256, 2, 16, 16), (64, 256, 1, 3, 3), (0, 1, 1)),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("case", CL_NATIVE_CASES, ids=lambda c: "x".join(map(str, c[0])) + "_w" + "x".join(map(str, c[1])))
def test_conv_channels_last_native_tiles(dev, case, dtype):
    """The MFMA tiles on channels-last input (atk_conv_fwd_prepacked_cl) against the same
    variant on the NC(D)HW copy: bit-identical (same patch values, same MFMA order), the
    output channels-last; one variant also against the float64 oracle.  Channels-last and
    contiguous weights give the same packed weights."""
    nat = _native()
    xs, ws, pad = case
    nd = len(xs) - 2
    x, w, b = _inputs(xs, ws, dtype, seed=sum(xs))
    fmt = torch.channels_last_3d if nd == 3 else torch.channels_last
    xd, wd, bd = x.to(dev), w.to(dev), b.to(dev)
    xcl = xd.contiguous(memory_format=fmt)
    plain = nat.conv3d if nd == 3 else nat.conv2d
    ran = 0
    for vi, name in _variants_for(dtype):
        if name == "direct":
            continue
        try:
            ycl = nat.conv_channels_last(xcl, wd, bd, 1, pad, 1, nd, variant=vi)
        except nat.Unsupported:
            continue
        assert ycl.is_contiguous(memory_format=fmt)
        try:
            y = plain(xd, wd, bd, 1, pad, 1, variant=vi)
        except nat.Unsupported:  # the NC(D)HW tile needs 16-byte rows along x: check values only
            y = None
        torch.cuda.synchronize()
        if y is not None:
            assert ycl.shape == y.shape and torch.equal(ycl.contiguous(), y), name
        if ran == 0 or y is None:
            ref = (O.conv3d if nd == 3 else O.conv2d)(x, w, b, 1, pad, 1)
            assert O.max_rel_err(ycl.float().contiguous().cpu(), ref) <= BAR[dtype], name
        if ran == 0:
            ycw = nat.conv_channels_last(xcl, wd.contiguous(memory_format=fmt), bd, 1, pad, 1, nd, variant=vi)
            assert torch.equal(ycw, ycl), name
        ran += 1
    assert ran >= 3


@pytest.mark.parametrize("case", CL_NATIVE_CASES, ids=lambda c: "x".join(map(str, c[0])) + "_w" + "x".join(map(str, c[1])))
def test_conv_channels_last_lds_staged_epilogue_bit_exact(dev, case, monkeypatch):
    """The channels-last LDS-staged epilogue (16-byte runs of 8 channels per position) stores the
    same bits as the per-value 8-byte stores it replaces (ATK_CONV_LDS_EPI=0), for every tile."""
    nat = _native()
    xs, ws, pad = case
    nd = len(xs) - 2
    x, w, b = _inputs(xs, ws, torch.bfloat16, seed=sum(xs) + 1)
    fmt = torch.channels_last_3d if nd == 3 else torch.channels_last
    xcl = x.to(dev).contiguous(memory_format=fmt)
    wd, bd = w.to(dev), b.to(dev)
    ran = 0
    for vi, name in _variants_for(torch.bfloat16):
        if name == "direct":
            continue
        try:
            monkeypatch.setenv("ATK_CONV_LDS_EPI", "0")
            want = nat.conv_channels_last(xcl, wd, bd, 1, pad, 1, nd, variant=vi)
            monkeypatch.delenv("ATK_CONV_LDS_EPI")
            got = nat.conv_channels_last(xcl, wd, bd, 1, pad, 1, nd, variant=vi)
        except nat.Unsupported:
            continue
        torch.cuda.synchronize()
        assert got.is_contiguous(memory_format=fmt)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), name
        ran += 1
    assert ran >= 3


def test_conv_channels_last_native_declines():
    """fp32, planes other than 3x3 / 7x7 and channel counts off multiples of 8 are declined
    (the dispatch then converts layouts for the NC(D)HW tiles)."""
    nat = _native()
    names = nat.variants(nat.OP_CONV)
    vi = names.index("h_w22_f22_cb32")
    for xs, ws, dt in [((1, 16, 4, 8, 8), (16, 16, 3, 3, 3), torch.float32),
                       ((1, 16, 4, 8, 8), (16, 16, 5, 5, 5), torch.bfloat16),
                       ((1, 12, 4, 8, 8), (16, 12, 3, 3, 3), torch.bfloat16)]:
        x = torch.randn(*xs, device="cuda", dtype=dt).contiguous(memory_format=torch.channels_last_3d)
        w = torch.randn(*ws, device="cuda", dtype=dt)
        vv = names.index("f32_w22_f22_cb16") if dt == torch.float32 else vi
        with pytest.raises(nat.Unsupported):
            nat.conv_channels_last(x, w, None, 1, 1, 1, 3, variant=vv)


TRANSPOSE_CASES = [
    # (B, R, C): vector path, odd rows / columns (element path), partial tiles, one row
    (2, 4096, 256), (1, 64, 64), (3, 100, 40), (2, 67, 13), (1, 1, 520), (5, 33, 1),
]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("case", TRANSPOSE_CASES, ids=lambda c: "x".join(map(str, c)))
def test_transpose_last2_bit_exact(dtype, case):
    """atk_transpose_last2 copies every element to its transposed place: bit-exact against
    torch's transpose on the same buffer, also from a misaligned base (element path)."""
    nat = _native()
    B, R, C = case
    g = torch.Generator().manual_seed(B * 131 + R * 7 + C)
    x = torch.randn(B * R * C + 1, generator=g).to(dtype).cuda()
    for base in (x[:-1], x[1:]):          # 16-byte aligned, then offset by one element
        out = torch.empty(B * C * R + 1, dtype=dtype, device="cuda")[1:]
        nat.transpose_last2(base, B, R, C, out)
        ref = base.view(B, R, C).transpose(1, 2).contiguous().view(-1)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16 if dtype != torch.float32 else torch.int32),
                           ref.view(torch.int16 if dtype != torch.float32 else torch.int32))


def test_transpose_last2_many_batches():
    """More batch entries than the grid's y extent (65535): the kernel strides over them."""
    nat = _native()
    B, R, C = 70000, 2, 8
    x = torch.arange(B * R * C, dtype=torch.float32, device="cuda").to(torch.bfloat16)
    out = torch.empty_like(x)
    nat.transpose_last2(x, B, R, C, out)
    assert torch.equal(out, x.view(B, R, C).transpose(1, 2).contiguous().view(-1))


@pytest.mark.parametrize("nd", [2, 3])
def test_channels_last_round_trip(nd):
    """channels_last_to_contiguous / contiguous_to_channels_last equal torch's
    .contiguous(memory_format=...) exactly, and round-trip."""
    nat = _native()
    shape = (2, 48, 5, 9, 11) if nd == 3 else (3, 40, 17, 19)
    fmt = torch.channels_last_3d if nd == 3 else torch.channels_last
    x = torch.randn(*shape, device="cuda").to(torch.bfloat16)
    xc = x.contiguous(memory_format=fmt)
    a = nat.channels_last_to_contiguous(xc)
    assert a.is_contiguous() and torch.equal(a, x)
    b = nat.contiguous_to_channels_last(a)
    assert b.is_contiguous(memory_format=fmt) and not b.is_contiguous()
    assert torch.equal(b, x) and b.stride() == xc.stride()


WGRAD_CASES = [
    # (N, Ci, Co, D, H, W, KD)
    (1, 32, 128, 4, 8, 16, 3),
    (2, 64, 128, 3, 5, 32, 3),     # H not a multiple of the 4-row stage
    (1, 32, 256, 1, 8, 64, 1),     # conv2d form
    (2, 32, 128, 2, 4, 48, 3),
    (2, 64, 256, 8, 20, 16, 3),    # 240 workgroups (XCD remap), chunks of 4 stages crossing planes
    (16, 32, 128, 1, 16, 64, 1),   # conv2d form, 16 chunks of 4 stages (XCD remap)
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", WGRAD_CASES)
def test_conv_wgrad_kernel_matches_float64(case, dtype):
    """atk_conv_wgrad against float64 aten.convolution_backward on the CPU (same quantised
    inputs): fp32 accumulation of exact 16-bit products, bar 1e-4 of the largest entry."""
    from amd_tuned_torch import _native
    N, Ci, Co, D, H, W, KD = case
    g = torch.Generator().manual_seed(Ci + Co + W)
    x = torch.randn(N, Ci, D, H, W, generator=g).to(dtype)
    dy = torch.randn(N, Co, D, H, W, generator=g).to(dtype)
    dw = _native.conv_wgrad(x.cuda(), dy.cuda(), KD)
    w = torch.zeros(Co, Ci, KD, 3, 3, dtype=torch.float64)
    ref = torch.ops.aten.convolution_backward(dy.double(), x.double(), w, None, [1, 1, 1], [KD // 2, 1, 1],
                                              [1, 1, 1], False, [0, 0, 0], 1, [False, True, False])[1]
    err = O.max_rel_err(dw, ref)
    assert err <= 1e-4, f"max_rel_err {err:.3g}"


def test_conv_wgrad_full_size_c5a():
    """C5a's shape (1, 256 -> 256, 8x64x64, k3) bf16 against fp32 aten on the GPU."""
    from amd_tuned_torch import _native
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(1, 256, 8, 64, 64, device="cuda", generator=g).to(torch.bfloat16)
    dy = torch.randn(1, 256, 8, 64, 64, device="cuda", generator=g).to(torch.bfloat16)
    dw = _native.conv_wgrad(x, dy, 3)
    w = torch.zeros(256, 256, 3, 3, 3, device="cuda")
    ref = torch.ops.aten.convolution_backward(dy.float(), x.float(), w, None, [1] * 3, [1] * 3, [1] * 3, False,
                                              [0] * 3, 1, [False, True, False])[1]
    assert O.max_rel_err(dw, ref) <= 1e-4


@pytest.mark.parametrize("channels_last", [False, True], ids=["ncdhw", "channels_last"])
@pytest.mark.parametrize("nd", [2, 3])
def test_conv_autograd_native_wgrad(nd, channels_last):
    """Weight and bias gradients through patched F.conv2d / F.conv3d (bf16) come from the
    native wgrad kernel and a reduction of dy, against float64 CPU autograd; channels-last
    input, weight and dy take the native layout conversions on the way."""
    import torch.nn.functional as F
    from amd_tuned_torch import _native
    calls = []
    orig = _native.conv_wgrad

    def spy(*a, **k):
        calls.append(1)
        return orig(*a, **k)
    _native.conv_wgrad = spy
    try:
        g = torch.Generator().manual_seed(nd)
        shape = (2, 32, 4, 8, 32) if nd == 3 else (2, 32, 16, 32)
        x = torch.randn(*shape, generator=g).to(torch.bfloat16)
        w = (torch.randn(128, 32, *([3] * nd), generator=g) * 0.05).to(torch.bfloat16)
        b = (torch.randn(128, generator=g) * 0.1).to(torch.bfloat16)
        conv = F.conv3d if nd == 3 else F.conv2d
        fmt = torch.channels_last_3d if nd == 3 else torch.channels_last
        lay = (lambda t: t.contiguous(memory_format=fmt)) if channels_last else (lambda t: t)
        xg, wg = (lay(t.cuda()).requires_grad_() for t in (x, w))
        bg = b.cuda().requires_grad_()
        y = conv(xg, wg, bg, 1, 1)
        if channels_last:
            assert y.is_contiguous(memory_format=fmt)
        dy = torch.randn(y.shape, generator=g).to(torch.bfloat16)
        y.backward(lay(dy.cuda()))
        xr, wr, br = (t.double().requires_grad_() for t in (x, w, b))
        import amd_tuned_torch
        amd_tuned_torch.disable()
        try:
            getattr(F, "conv3d" if nd == 3 else "conv2d")(xr, wr, br, 1, 1).backward(dy.double())
        finally:
            amd_tuned_torch.enable()
    finally:
        _native.conv_wgrad = orig
    assert calls, "native wgrad not used"
    assert O.max_rel_err(wg.grad.float(), wr.grad) <= 1e-2
    assert O.max_rel_err(bg.grad.float(), br.grad) <= 1e-2
    assert O.max_rel_err(xg.grad.float(), xr.grad) <= 1e-2


# ---------------------------------------------------------------------------
# packed weights kept across calls (atk_conv_pack_weights / atk_conv_fwd_prepacked)
# ---------------------------------------------------------------------------
def _raw_conv3d(nat, x, w, b, s, p, d, vi):
    """atk_conv_fwd (packing inside the call) with no cache in between."""
    import ctypes
    L = nat.lib()
    dt = nat._DTYPE_CODE[x.dtype]
    N, Ci, D, H, W = x.shape
    Co, _, KD, KH, KW = w.shape
    geom = (N, Ci, D, H, W, Co, KD, KH, KW, *([s] * 3), *([p] * 3), *([d] * 3))
    y = torch.empty(N, Co, *[(e + 2 * p - d * (k - 1) - 1) // s + 1 for e, k in zip((D, H, W), (KD, KH, KW))],
                    dtype=x.dtype, device=x.device)
    nbytes = L.atk_conv_workspace_bytes(*geom, dt, vi)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
    rc = L.atk_conv_fwd(x.data_ptr(), w.data_ptr(), None if b is None else b.data_ptr(), y.data_ptr(), *geom, dt,
                        vi, ws.data_ptr(), ctypes.c_size_t(ws.numel()), torch.cuda.current_stream().cuda_stream)
    assert rc == 0, nat.last_error()
    return y


@pytest.mark.parametrize("xs,ws", [((1, 32, 8, 16, 16), (64, 32, 3, 3, 3)),      # split-K tiles
                                   ((1, 64, 16, 32, 32), (64, 64, 3, 3, 3)),      # config 4, small
                                   ((2, 5, 5, 6, 7), (3, 5, 3, 3, 3))])           # off the tiles
def test_prepacked_conv_equals_single_call(dev, xs, ws):
    """For every 16-bit MFMA variant that takes the shape, the cached-packed-weight path gives
    exactly the bytes of the pack-in-the-call path."""
    nat = _native()
    x, w, b = _inputs(xs, ws, torch.bfloat16, seed=3)
    xd, wd, bd = x.to(dev), w.to(dev), b.to(dev)
    ran = 0
    for vi, name in _variants_for(torch.bfloat16):
        if name == "direct":
            continue
        try:
            want = _raw_conv3d(nat, xd, wd, bd, 1, 1, 1, vi)
        except AssertionError:
            continue  # the variant declines the shape
        got = nat.conv3d(xd, wd, bd, 1, 1, 1, variant=vi)
        again = nat.conv3d(xd, wd, bd, 1, 1, 1, variant=vi)  # from the cache
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), name
        assert torch.equal(again.view(torch.int16), want.view(torch.int16)), name
        ran += 1
    assert ran >= 3


def test_packed_weight_cache_follows_the_weight(dev):
    """A cached entry serves the same weight object while its contents are unchanged; an
    in-place update (version bump) is packed again; the entry dies with the weight."""
    import gc
    nat = _native()
    nat.clear_packed_weight_cache()
    x, w, b = _inputs((1, 32, 8, 16, 16), (64, 32, 3, 3, 3), torch.float16, seed=4)
    xd, wd = x.to(dev), w.to(dev)
    vi = [i for i, n in _variants_for(torch.float16) if n == "h_w22_f22_cb32"][0]
    y1 = nat.conv3d(xd, wd, None, 1, 1, 1, variant=vi)
    assert nat.packed_weight_cache_size() == 1
    nat.conv3d(xd, wd, None, 1, 1, 1, variant=vi)
    assert nat.packed_weight_cache_size() == 1                 # hit, nothing new
    wd.mul_(2.0)                                               # in place: new version
    y2 = nat.conv3d(xd, wd, None, 1, 1, 1, variant=vi)
    torch.cuda.synchronize()
    assert torch.equal(y2.cpu(), (2.0 * y1.float()).to(torch.float16).cpu()) or \
        O.max_rel_err(y2.cpu(), O.conv3d(x, 2.0 * w.float(), None, 1, 1, 1)) <= 1e-2
    assert O.max_rel_err(y2.cpu(), O.conv3d(x, (2.0 * w.float()).to(torch.float16), None, 1, 1, 1)) <= 1e-2
    del wd
    gc.collect()
    assert nat.packed_weight_cache_size() == 0                 # entries die with the weight


LDS_EPI_CASES = [
    # one K stage (never split K): every 16-bit tile's plain epilogue runs; rows partly
    # outside the output (H = 10), depth and 2-D shapes
    ((1, 16, 4, 10, 64), (64, 16, 1, 3, 3)),
    ((2, 16, 3, 16, 32), (96, 16, 1, 3, 3)),
    ((2, 16, 12, 64), (32, 16, 3, 3)),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("case", LDS_EPI_CASES, ids=lambda c: "x".join(map(str, c[0])))
def test_conv_lds_staged_epilogue_bit_exact(dev, case, dtype, monkeypatch):
    """The LDS-staged epilogue (16-byte runs of 8 positions per channel) stores the same bits as
    the per-value stores it replaces (ATK_CONV_LDS_EPI=0), for every 16-bit tile, and both
    match the float64 oracle."""
    xs, ws = case
    nat = _native()
    x, w, b = _inputs(xs, ws, dtype, seed=11)
    conv = nat.conv3d if len(xs) == 5 else nat.conv2d
    ref = (O.conv3d if len(xs) == 5 else O.conv2d)(x, w, b, 1, (0, 1, 1) if len(xs) == 5 else 1, 1)
    pad = (0, 1, 1) if len(xs) == 5 else 1
    xd, wd, bd = x.to(dev), w.to(dev), b.to(dev)
    ran = 0
    for vi, name in _variants_for(dtype):
        try:
            monkeypatch.setenv("ATK_CONV_LDS_EPI", "0")
            want = conv(xd, wd, bd, 1, pad, 1, variant=vi)
            monkeypatch.delenv("ATK_CONV_LDS_EPI")
            got = conv(xd, wd, bd, 1, pad, 1, variant=vi)
        except nat.Unsupported:
            continue
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), name
        assert O.max_rel_err(got.cpu(), ref) <= BAR[dtype], name
        ran += 1
    assert ran >= 5
