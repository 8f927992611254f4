"""GPU parity of the conv epilogue fusion: residual add and GroupNorm statistics written by the
MFMA conv's epilogue (atk_conv_fwd_prepacked_ex), and the GroupNorm apply pass that consumes
them (atk_group_norm_apply), against the float64 oracle.  Bars: fp32 <= 1e-5 (conv),
fp16/bf16 <= 1e-2 max-abs-rel; GroupNorm of the stored conv output <= 1e-2 (16-bit) /
1e-5 (fp32)."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O

pytestmark = pytest.mark.gpu

BAR = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 1e-2}
GN_BAR = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 1e-2}


def _native():
    from amd_tuned_torch import _native
    return _native


def _inputs(xs, ws, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*xs, generator=g)
    w = torch.randn(*ws, generator=g) * math.sqrt(2.0 / math.prod(ws[1:]))
    b = 0.3 * torch.randn(ws[0], generator=g)
    return x.to(dtype), w.to(dtype), b.to(dtype)


def _mfma(nat, dtype):
    pre = "f32_" if dtype == torch.float32 else "h_"
    return [(i, n) for i, n in enumerate(nat.variants(nat.OP_CONV)) if n.startswith(pre)]


def _merge(records: np.ndarray):
    """(mean, var) per (n, g) from [N*G][P][4] records (count, mean, M2, -), float64."""
    n, m, m2 = records[..., 0], records[..., 1], records[..., 2]
    cnt = n.sum(-1)
    mean = (n * m).sum(-1) / cnt
    var = (m2 + n * (m - mean[:, None]) ** 2).sum(-1) / cnt
    return cnt, mean, var


CASES = [
    # xshape, wshape, pad, groups (channels per group = Co / groups)
    ((1, 32, 8, 16, 16), (64, 32, 3, 3, 3), 1, 8),     # cpg 8
    ((2, 16, 5, 9, 16), (32, 16, 3, 3, 3), 1, 8),      # cpg 4, edge tiles (H = 9, D = 5), N = 2
    ((1, 32, 4, 12, 24), (64, 32, 3, 3, 3), 1, 4),     # cpg 16
    ((1, 32, 4, 8, 8), (64, 32, 3, 3, 3), 1, 2),       # cpg 32
    ((1, 16, 4, 8, 8), (128, 16, 3, 3, 3), 1, 2),      # cpg 64: a group spans two 32-blocks
    ((1, 16, 16, 64, 64), (32, 16, 3, 3, 3), 1, 4),    # large enough that fp32 tiles do not split
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c[0])) + "_g%d" % c[3])
def test_conv_epilogue_group_norm_records(dev, case, dtype):
    """Every unsplit MFMA variant: y is the plain conv's output byte for byte, the records merge
    to the statistics of the stored y (float64), and the apply pass is GroupNorm(+SiLU) of y."""
    xs, ws, pad, G = case
    nat = _native()
    x, w, b = _inputs(xs, ws, dtype, seed=sum(xs) + G)
    xd, wd, bd = x.to(dev), w.to(dev), b.to(dev)
    gc = torch.Generator().manual_seed(5)
    gm = (1 + 0.1 * torch.randn(ws[0], generator=gc)).to(dtype)
    bt = (0.1 * torch.randn(ws[0], generator=gc)).to(dtype)
    ran = 0
    for vi, name in _mfma(nat, dtype):
        try:
            y, rec, nrec = nat.conv_gn_stats(xd, wd, bd, 1, pad, 1, 3, G, variant=vi)
        except nat.Unsupported:
            continue  # declines the shape, or splits it
        plain = nat.conv3d(xd, wd, bd, 1, pad, 1, variant=vi)
        torch.cuda.synchronize()
        assert torch.equal(y, plain), name
        assert O.max_rel_err(y.cpu(), O.conv3d(x, w, b, 1, pad, 1)) <= BAR[dtype], name
        yc = y.cpu().double().reshape(xs[0] * G, -1)
        r = rec.cpu().double().numpy().reshape(xs[0] * G, nrec, 4)
        cnt, mean, var = _merge(r)
        assert np.array_equal(cnt, np.full(xs[0] * G, yc.shape[1], dtype=np.float64)), name
        ref_mean = yc.mean(-1).numpy()
        ref_var = yc.var(-1, unbiased=False).numpy()
        scale = max(1.0, float(np.abs(ref_mean).max()))
        assert np.abs(mean - ref_mean).max() <= 1e-5 * scale + 1e-6, name
        assert np.abs(var - ref_var).max() <= 1e-4 * ref_var.max() + 1e-7, name
        if (y.numel() // (y.shape[0] * y.shape[1])) % (16 // y.element_size()):
            # the apply pass reads 16-byte vectors: a spatial size off that grid is declined
            # (the fused block then runs stock)
            with pytest.raises(nat.Unsupported):
                nat.group_norm_apply(y, G, gm.to(dev), bt.to(dev), 1e-5, rec, nrec)
            ran += 1
            continue
        for silu in (False, True):
            out = nat.group_norm_apply(y, G, gm.to(dev), bt.to(dev), 1e-5, rec, nrec, silu=silu)
            torch.cuda.synchronize()
            ref = O.group_norm(y.cpu(), G, gm, bt, 1e-5, silu=silu)
            assert O.max_rel_err(out.cpu(), ref) <= GN_BAR[dtype], (name, silu)
        ran += 1
    # the fp32 tiles split K on the small shapes (too few output tiles), which rules the
    # epilogue out there; the last case is large enough for them
    assert ran >= 1 or (dtype == torch.float32 and xs[2] * xs[3] * xs[4] < 32768)


def test_conv_epilogue_needs_aligned_rows(dev):
    """The epilogue instantiations read input rows as 16-byte vectors: a width off that grid
    (W = 11 for bf16) is declined with ATK_UNSUPPORTED, and the plain conv still serves it."""
    nat = _native()
    x, w, b = _inputs((2, 16, 5, 9, 11), (32, 16, 3, 3, 3), torch.bfloat16, seed=3)
    xd, wd, bd = x.to(dev), w.to(dev), b.to(dev)
    for vi, name in _mfma(nat, torch.bfloat16):
        try:
            nat.conv3d(xd, wd, bd, 1, 1, 1, variant=vi)
        except nat.Unsupported:
            continue
        with pytest.raises(nat.Unsupported):
            nat.conv_gn_stats(xd, wd, bd, 1, 1, 1, 3, 8, variant=vi)
        with pytest.raises(nat.Unsupported):
            nat.conv3d(xd, wd, bd, 1, 1, 1, variant=vi, residual=torch.zeros(2, 32, 5, 9, 11, device=dev,
                                                                            dtype=torch.bfloat16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_conv_epilogue_residual(dev, dtype):
    """y = conv + bias + residual in the epilogue, for every MFMA variant that takes the shape
    unsplit, against the float64 oracle; conv2d too."""
    nat = _native()
    x, w, b = _inputs((2, 16, 8, 64, 64), (48, 16, 3, 3, 3), dtype, seed=8)  # unsplit for fp32 tiles too
    r = torch.randn(2, 48, 8, 64, 64, generator=torch.Generator().manual_seed(9)).to(dtype)
    ref = O.conv3d(x, w, b, 1, 1, 1) + O.f64(r)
    xd, wd, bd, rd = x.to(dev), w.to(dev), b.to(dev), r.to(dev)
    ran = 0
    for vi, name in _mfma(nat, dtype):
        try:
            y = nat.conv3d(xd, wd, bd, 1, 1, 1, variant=vi, residual=rd)
        except nat.Unsupported:
            continue
        torch.cuda.synchronize()
        assert O.max_rel_err(y.cpu(), ref) <= max(BAR[dtype], 2e-5), name
        ran += 1
    assert ran >= 1
    x2, w2, b2 = _inputs((4, 16, 96, 128), (32, 16, 3, 3), dtype, seed=10)
    r2 = torch.randn(4, 32, 96, 128, generator=torch.Generator().manual_seed(11)).to(dtype)
    ref2 = O.conv2d(x2, w2, b2, 1, 1, 1) + O.f64(r2)
    for vi, name in _mfma(nat, dtype):
        try:
            y2 = nat.conv2d(x2.to(dev), w2.to(dev), b2.to(dev), 1, 1, 1, variant=vi, residual=r2.to(dev))
        except nat.Unsupported:
            continue
        torch.cuda.synchronize()
        assert O.max_rel_err(y2.cpu(), ref2) <= max(BAR[dtype], 2e-5), name


def test_conv_residual_api(dev):
    """conv_fusion_ops.conv_residual through its contest (cached winner on the second call)
    equals the stock conv plus the residual within the bf16 bar."""
    from amd_tuned_torch import conv_fusion_ops
    x, w, b = _inputs((1, 64, 8, 32, 32), (64, 64, 3, 3, 3), torch.bfloat16, seed=12)
    r = torch.randn(1, 64, 8, 32, 32, generator=torch.Generator().manual_seed(13)).to(torch.bfloat16)
    ref = O.conv3d(x, w, b, 1, 1, 1) + O.f64(r)
    xd, wd, bd, rd = x.to(dev), w.to(dev), b.to(dev), r.to(dev)
    with torch.no_grad():
        for _ in range(2):
            y = conv_fusion_ops.conv_residual(xd, wd, bd, rd, 1, 1, 1)
            torch.cuda.synchronize()
            assert O.max_rel_err(y.cpu(), ref) <= 1e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_fused_conv_group_norm_silu_block(dev, dtype):
    """The config-5 block order (Conv3d -> GroupNorm -> SiLU) through FusedConvGroupNormSiLU and
    through the patched nn.Sequential at inference: the conv epilogue's statistics path, against
    the float64 CPU block."""
    import amd_tuned_torch  # noqa: F401
    from amd_tuned_torch import conv_fusion_ops
    torch.manual_seed(14)
    conv = torch.nn.Conv3d(64, 64, 3, padding=1)
    norm = torch.nn.GroupNorm(32, 64, eps=1e-6)
    with torch.no_grad():
        norm.weight.normal_(1.0, 0.1)
        norm.bias.normal_(0.0, 0.1)
    x = torch.randn(1, 64, 4, 32, 32)
    seq = torch.nn.Sequential(conv, norm, torch.nn.SiLU()).to(dev, dtype)
    # the float64 reference runs on the same (rounded) input and parameters as the GPU block
    p64 = [t.detach().cpu().double() for t in (seq[0].weight, seq[0].bias, seq[1].weight, seq[1].bias)]
    with torch.no_grad():
        ref = conv_fusion_ops._dispatch_stock_gn()(
            amd_tuned_torch._dispatch._STOCK_F["conv3d"](x.to(dtype).double(), p64[0], p64[1], 1, 1),
            32, p64[2], p64[3], 1e-6)
        ref = F.silu(ref)
    fused = conv_fusion_ops.FusedConvGroupNormSiLU(seq[0], seq[1])
    xd = x.to(dev, dtype)
    bar = BAR[dtype]
    with torch.no_grad():
        for _ in range(2):   # contest, then the cached winner
            y = fused(xd)
            torch.cuda.synchronize()
            assert O.max_rel_err(y.cpu(), ref) <= bar
        y2 = seq(xd)
        torch.cuda.synchronize()
        assert O.max_rel_err(y2.cpu(), ref) <= bar


def test_conv_gn_stats_and_apply_full_size_c5(dev):
    """Config 5's block at full size ([1, 256, 8, 64, 64] bf16, 3x3x3, GroupNorm(32, eps 1e-6)
    + SiLU) through the fused path -- conv epilogue statistics, then the apply pass -- for
    every MFMA variant that takes it unsplit: 4096 sampled conv outputs against the float64
    oracle, the merged records against the float64 statistics of the stored output, and the
    whole GroupNorm+SiLU output against the float64 oracle of GroupNorm+SiLU on that output."""
    nat = _native()
    xs, ws, G, eps = (1, 256, 8, 64, 64), (256, 256, 3, 3, 3), 32, 1e-6
    x, w, b = _inputs(xs, ws, torch.bfloat16, seed=1005)
    gc = torch.Generator().manual_seed(6)
    gm = (1 + 0.1 * torch.randn(256, generator=gc)).to(torch.bfloat16)
    bt = (0.1 * torch.randn(256, generator=gc)).to(torch.bfloat16)
    pts = torch.randint(0, math.prod(xs[:1]) * 256 * 8 * 64 * 64, (4096,), generator=gc).numpy()
    ref_pts = O.conv3d(x, w, b, 1, 1, 1, points=pts)
    xd, wd, bd = x.to(dev), w.to(dev), b.to(dev)
    ran = 0
    for vi, name in _mfma(nat, torch.bfloat16):
        try:
            y, rec, nrec = nat.conv_gn_stats(xd, wd, bd, 1, 1, 1, 3, G, variant=vi)
        except nat.Unsupported:
            continue
        out = nat.group_norm_apply(y, G, gm.to(dev), bt.to(dev), eps, rec, nrec, silu=True)
        torch.cuda.synchronize()
        yp = y.flatten()[torch.from_numpy(pts).to(dev)].cpu()
        assert float(np.max(np.abs(O.f64(yp) - ref_pts)) / np.max(np.abs(ref_pts))) <= 1e-2, name
        yd = y.double().reshape(G, -1)
        r = rec.cpu().double().numpy().reshape(G, nrec, 4)
        cnt, mean, var = _merge(r)
        ref_mean = yd.mean(-1).cpu().numpy()
        ref_var = yd.var(-1, unbiased=False).cpu().numpy()
        assert np.array_equal(cnt, np.full(G, yd.shape[1], dtype=np.float64)), name
        assert np.abs(mean - ref_mean).max() <= 1e-5 * max(1.0, float(np.abs(ref_mean).max())) + 1e-6, name
        assert np.abs(var - ref_var).max() <= 1e-4 * ref_var.max() + 1e-7, name
        ref = O.group_norm(y.cpu(), G, gm, bt, eps, silu=True)
        assert O.max_rel_err(out.cpu(), ref) <= 1e-2, name
        ran += 1
        del y, rec, out, yd
    assert ran >= 1


ONEPASS_CASES = [
    # xshape, wshape, pad, groups, silu, affine
    ((1, 32, 8, 16, 16), (64, 32, 3, 3, 3), 1, 8, True, True),      # cpg 8
    ((2, 16, 5, 9, 16), (32, 16, 3, 3, 3), 1, 8, False, True),     # cpg 4, edge tiles, N = 2
    ((1, 32, 4, 12, 24), (64, 32, 3, 3, 3), 1, 4, True, False),    # cpg 16, no affine
    ((1, 32, 4, 8, 8), (64, 32, 3, 3, 3), 1, 2, True, True),       # cpg 32
    ((1, 16, 4, 8, 8), (128, 16, 3, 3, 3), 1, 2, False, True),     # cpg 64: two 32-channel parts
    ((2, 64, 4, 32, 32), (128, 64, 3, 3, 3), 1, 32, True, True),   # cpg 4 over 128 channels, N = 2
    ((1, 32, 2, 16, 16), (64, 32, 1, 7, 7), (0, 3, 3), 16, True, True),  # 7x7 plane
]


def _onepass_params(co, dtype, affine, seed):
    if not affine:
        return None, None
    gc = torch.Generator().manual_seed(seed)
    return (1 + 0.1 * torch.randn(co, generator=gc)).to(dtype), (0.1 * torch.randn(co, generator=gc)).to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("case", ONEPASS_CASES, ids=lambda c: "x".join(map(str, c[0])) + "_g%d" % c[3])
def test_conv_group_norm_one_pass(dev, case, dtype):
    """Conv -> GroupNorm (-> SiLU) in one cooperative launch, for every 16-bit variant that
    takes the shape: against the float64 oracle of GroupNorm(+SiLU) applied to the plain conv's
    output of the same variant (the statistics are of that stored output), and against the
    float64 oracle of the whole block (bar 1e-2); repeats are bit-identical and no wait ran out."""
    xs, ws, pad, G, silu, affine = case
    nat = _native()
    x, w, b = _inputs(xs, ws, dtype, seed=sum(xs) + 7 * G)
    gm, bt = _onepass_params(ws[0], dtype, affine, seed=G)
    xd, wd, bd = x.to(dev), w.to(dev), b.to(dev)
    gmd = gm.to(dev) if gm is not None else None
    btd = bt.to(dev) if bt is not None else None
    block_ref = O.group_norm(torch.from_numpy(O.conv3d(x, w, b, 1, pad, 1)).to(dtype), G, gm, bt, 1e-5, silu=silu)
    ran = 0
    for vi, name in _mfma(nat, dtype):
        try:
            out = nat.conv_group_norm(xd, wd, bd, gmd, btd, 1, pad, 1, 3, G, 1e-5, silu=silu, variant=vi)
        except nat.Unsupported:
            continue
        plain = nat.conv3d(xd, wd, bd, 1, pad, 1, variant=vi)
        again = nat.conv_group_norm(xd, wd, bd, gmd, btd, 1, pad, 1, 3, G, 1e-5, silu=silu, variant=vi)
        torch.cuda.synchronize()
        assert not nat.conv_group_norm_wait_error(dev), name
        assert torch.equal(out.view(torch.int16), again.view(torch.int16)), name
        ref = O.group_norm(plain.cpu(), G, gm, bt, 1e-5, silu=silu)
        assert O.max_rel_err(out.cpu(), ref) <= GN_BAR[dtype], name
        assert O.max_rel_err(out.cpu(), block_ref) <= 1e-2, name
        ran += 1
    assert ran >= 1


def test_conv_group_norm_one_pass_graph_replay(dev):
    """The one-pass launch captured in a HIP graph: six replays, each after the input changed
    in place, against eager calls on the same inputs (the slot tags come from the epoch the
    launch itself advances, so a replay never reads the previous replay's records)."""
    nat = _native()
    xs, ws, G = (1, 32, 8, 16, 16), (64, 32, 3, 3, 3), 8
    x, w, b = _inputs(xs, ws, torch.bfloat16, seed=77)
    gm, bt = _onepass_params(64, torch.bfloat16, True, seed=3)
    xd, wd, bd, gmd, btd = x.to(dev), w.to(dev), b.to(dev), gm.to(dev), bt.to(dev)
    out = torch.empty(1, 64, 8, 16, 16, dtype=torch.bfloat16, device=dev)
    vi = None
    for i, _ in _mfma(nat, torch.bfloat16):
        try:  # (also the warm-up: packed weights and workspace exist before the capture)
            nat.conv_group_norm(xd, wd, bd, gmd, btd, 1, 1, 1, 3, G, 1e-6, silu=True, variant=i, out=out)
        except nat.Unsupported:
            continue
        vi = i
        break
    assert vi is not None
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            nat.conv_group_norm(xd, wd, bd, gmd, btd, 1, 1, 1, 3, G, 1e-6, silu=True, variant=vi, out=out)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.Generator().manual_seed(78)
    for _ in range(6):
        xd.copy_(torch.randn(*xs, generator=g).to(torch.bfloat16))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = nat.conv_group_norm(xd, wd, bd, gmd, btd, 1, 1, 1, 3, G, 1e-6, silu=True, variant=vi)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    assert not nat.conv_group_norm_wait_error(dev)


def test_conv_group_norm_one_pass_full_size_c5(dev):
    """Config 5's block at full size ([1, 256, 8, 64, 64] bf16, 3x3x3, GroupNorm(32, eps 1e-6)
    + SiLU) in one launch, for every variant that takes it: against the float64 oracle of
    GroupNorm+SiLU on the same variant's plain conv output."""
    nat = _native()
    xs, ws, G, eps = (1, 256, 8, 64, 64), (256, 256, 3, 3, 3), 32, 1e-6
    x, w, b = _inputs(xs, ws, torch.bfloat16, seed=1005)
    gm, bt = _onepass_params(256, torch.bfloat16, True, seed=6)
    xd, wd, bd, gmd, btd = x.to(dev), w.to(dev), b.to(dev), gm.to(dev), bt.to(dev)
    ran = 0
    for vi, name in _mfma(nat, torch.bfloat16):
        try:
            out = nat.conv_group_norm(xd, wd, bd, gmd, btd, 1, 1, 1, 3, G, eps, silu=True, variant=vi)
        except nat.Unsupported:
            continue
        plain = nat.conv3d(xd, wd, bd, 1, 1, 1, variant=vi)
        torch.cuda.synchronize()
        assert not nat.conv_group_norm_wait_error(dev), name
        ref = O.group_norm(plain.cpu(), G, gm, bt, eps, silu=True)
        assert O.max_rel_err(out.cpu(), ref) <= 1e-2, name
        ran += 1
        del out, plain
    assert ran >= 1
