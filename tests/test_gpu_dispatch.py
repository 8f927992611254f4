"""GPU tests of the patched API around the kernels: BASELINE config 1's workload, the
depthwise training path at widths the weight-gradient kernel does not take, the
reference-shape causal mode, the MIOpen rescue, torch.compile routing and scratch isolation
between streams.  Parity against the float64 oracle with the north-star bars (fp32 <= 1e-5,
fp16/bf16 <= 1e-2 max-abs-rel)."""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O

pytestmark = pytest.mark.gpu

BAR = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 1e-2}


def _att():
    import amd_tuned_torch
    return amd_tuned_torch


def _config1(seed=1000):
    """x [8,256,2048] ~ N(0,1), w [256,1,3] ~ N(0,1/3), b ~ N(0,0.1)
    (second argument = variance), seeded, drawn in fp32 on the CPU."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(8, 256, 2048, generator=g)
    w = torch.randn(256, 1, 3, generator=g) * (1.0 / 3.0) ** 0.5
    b = torch.randn(256, generator=g) * 0.1 ** 0.5
    return x, w, b


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["fp32", "fp16"])
def test_config1_workload_on_the_hip_kernel(dev, dtype):
    """Config 1's depthwise conv1d ([8,256,2048], k3, p1) on every native variant that takes
    it and through the patched F.conv1d, against the oracle (fp32 <= 1e-5, fp16 <= 1e-2)."""
    att = _att()
    nat = att._native
    x, w, b = _config1()
    x, w, b = x.to(dtype), w.to(dtype), b.to(dtype)
    ref = O.dwconv1d(x, w.squeeze(1), b, 1, 2048)
    xd, wd, bd = x.to(dev), w.to(dev), b.to(dev)
    ran = 0
    for vi, name in enumerate(nat.variants(nat.OP_DWCONV1D)):
        try:
            y = nat.dwconv1d(xd, wd.squeeze(1), bd, 1, 2048, variant=vi)
        except nat.Unsupported:
            continue
        torch.cuda.synchronize()
        err = O.max_rel_err(y.cpu(), ref)
        assert err <= BAR[dtype], f"{name}: {err:.3g}"
        ran += 1
    assert ran >= 3
    y = F.conv1d(xd, wd, bd, padding=1, groups=256)
    torch.cuda.synchronize()
    assert O.max_rel_err(y.cpu(), ref) <= BAR[dtype]


def test_config1_cpu_path_is_bit_exact_stock():
    """Config 1 as the reference states it: on the CPU the patched F.conv1d is stock, bit for
    bit (repeated here so the GPU run carries it)."""
    att = _att()
    x, w, b = _config1()
    stock = att.miopen_fallback._original_conv1d
    assert stock is not None and F.conv1d is not stock
    assert torch.equal(F.conv1d(x, w, b, padding=1, groups=256), stock(x, w, b, 1, 1, 1, 256))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_depthwise_autograd_k7_same_keeps_native_dx(dev, dtype, monkeypatch):
    """K = 7 'same' (padding 3) through the patched F.conv1d with gradients: the weight-
    gradient kernel declines K > 5, dx must still come from the native kernel and every
    gradient must match the oracle."""
    att = _att()
    nat = att._native
    calls = []
    real = nat.dwconv1d
    monkeypatch.setattr(nat, "dwconv1d", lambda *a, **k: calls.append(a[0].shape) or real(*a, **k))
    g = torch.Generator().manual_seed(77)
    N, C, L, K, pad = 2, 8, 257, 7, 3
    x = torch.randn(N, C, L, generator=g).to(dtype)
    w = (torch.randn(C, K, generator=g) * K ** -0.5).to(dtype)
    b = (0.3 * torch.randn(C, generator=g)).to(dtype)
    dy = torch.randn(N, C, L, generator=g).to(dtype)
    xd = x.to(dev).requires_grad_(True)
    wd = w.to(dev).unsqueeze(1).requires_grad_(True)
    bd = b.to(dev).requires_grad_(True)
    y = F.conv1d(xd, wd, bd, padding=pad, groups=C)   # first call: the contest runs every variant
    assert O.max_rel_err(y.detach().cpu(), O.dwconv1d(x, w, b, pad, L)) <= BAR[dtype]
    calls.clear()
    gx, gw, gb = torch.autograd.grad(y, (xd, wd, bd), dy.to(dev))
    rdx, rdw, rdb = O.dwconv1d_bwd(x, w, dy, pad)
    assert O.max_rel_err(gx.cpu(), rdx) <= BAR[dtype]
    assert O.max_rel_err(gw.cpu().reshape(C, K), rdw) <= max(BAR[dtype], 1e-4)
    assert O.max_rel_err(gb.cpu(), rdb) <= max(BAR[dtype], 1e-4)
    # the backward ran the input gradient as the forward kernel on dy, once
    assert calls == [(N, C, L)]
    direct = nat.dwconv1d_backward(dy.to(dev), x.to(dev), w.to(dev), pad, (True, True, True))
    assert direct[0] is not None and direct[1] is None and direct[2] is None


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_causal_truncate_mode_returns_length_l(dev, dtype, monkeypatch):
    """AMD_TUNED_TORCH_CAUSAL_CONV1D_TRUNCATE=1: F.conv1d(x, w, b, padding=K-1, groups=C) with
    K in 2..4 returns the causal length-L output (the reference's shape), equal to stock's
    output cut to L; other widths keep stock's shape."""
    att = _att()
    monkeypatch.setattr(att.miopen_fallback, "_CAUSAL_TRUNCATE", True)
    g = torch.Generator().manual_seed(5)
    N, C, L = 2, 16, 1000
    for K in (2, 3, 4, 5):
        x = torch.randn(N, C, L, generator=g).to(dtype)
        w = (torch.randn(C, 1, K, generator=g) * 0.5).to(dtype)
        b = (0.1 * torch.randn(C, generator=g)).to(dtype)
        y = F.conv1d(x.to(dev), w.to(dev), b.to(dev), padding=K - 1, groups=C)
        torch.cuda.synchronize()
        ref = O.dwconv1d(x, w.squeeze(1), b, K - 1, L + K - 1)
        if K <= 4:
            assert tuple(y.shape) == (N, C, L)
            ref = ref[..., :L]
        else:
            assert tuple(y.shape) == (N, C, L + K - 1)
        assert O.max_rel_err(y.cpu(), ref) <= BAR[dtype]


def test_miopen_rescue_on_gpu_input(dev, monkeypatch):
    """A GPU conv whose stock call fails with a miopenStatus error is retried after
    torch.cuda.empty_cache(); when that fails too it runs on the CPU in fp32 and comes back
    to the GPU in the input's dtype."""
    att = _att()
    stock = att.miopen_fallback._original_conv1d
    g = torch.Generator().manual_seed(9)
    x = torch.randn(2, 4, 64, generator=g).to(torch.float16).to(dev)
    w = torch.randn(6, 4, 3, generator=g).to(torch.float16).to(dev)
    emptied = []
    real_empty = torch.cuda.empty_cache
    monkeypatch.setattr(torch.cuda, "empty_cache", lambda: emptied.append(1) or real_empty())
    seen = []

    def failing_on_gpu(inp, *rest):
        seen.append(inp.device.type)
        if inp.is_cuda:
            raise RuntimeError("miopenStatusUnknownError")
        return stock(inp, *rest)
    y = att.miopen_fallback._miopen_safe_conv("conv1d", failing_on_gpu)(x, w, None, 1, 1)
    assert seen == ["cuda", "cuda", "cpu"] and emptied == [1]
    assert y.is_cuda and y.dtype == torch.float16
    ref = stock(x.float().cpu(), w.float().cpu(), None, 1, 1).half()
    assert torch.equal(y.cpu(), ref)


def test_torch_compile_block_matches_oracle_without_graph_breaks(dev):
    """torch.compile of conv3d -> GroupNorm -> GroupNorm+SiLU and a depthwise conv1d, forward
    and backward (AOTAutograd, eager kernels): one graph, no breaks, the amd_tuned_torch ops in
    it, outputs and gradients against the float64 oracle / float64 stock autograd."""
    import torch._dynamo
    att = _att()
    torch._dynamo.reset()
    g = torch.Generator().manual_seed(31)
    dt = torch.bfloat16
    x = torch.randn(1, 16, 4, 16, 16, generator=g).to(dt)
    w3 = (torch.randn(16, 16, 3, 3, 3, generator=g) * (2.0 / (16 * 27)) ** 0.5).to(dt)
    b3 = (0.1 * torch.randn(16, generator=g)).to(dt)
    gm = (1 + 0.1 * torch.randn(16, generator=g)).to(dt)
    bt = (0.1 * torch.randn(16, generator=g)).to(dt)
    x1 = torch.randn(2, 32, 512, generator=g).to(dt)
    w1 = (0.5 * torch.randn(32, 1, 4, generator=g)).to(dt)
    b1 = (0.1 * torch.randn(32, generator=g)).to(dt)

    def block(x, w3, b3, gm, bt, x1, w1, b1):
        y = F.conv3d(x, w3, b3, 1, 1)
        y = F.group_norm(y, 4, gm, bt, 1e-5)
        y = att.group_norm_silu(y, 4, gm, bt, 1e-5)
        z = F.conv1d(x1, w1, b1, padding=3, groups=32)
        return y, z

    dev_args = [t.to(dev) for t in (x, w3, b3, gm, bt, x1, w1, b1)]
    explain = torch._dynamo.explain(block)(*dev_args)
    assert explain.graph_break_count == 0 and explain.graph_count == 1
    names = " ".join(str(n.target) for gmod in explain.graphs for n in gmod.graph.nodes)
    for op in ("conv3d_native", "group_norm", "group_norm_silu", "depthwise_conv1d_forward"):
        assert "amd_tuned_torch.%s" % op in names

    torch._dynamo.reset()
    compiled = torch.compile(block, backend="aot_eager", fullgraph=True)
    # inference: forward only
    with torch.no_grad():
        y, z = compiled(*dev_args)
    torch.cuda.synchronize()
    h = F.conv3d(x.double(), w3.double(), b3.double(), 1, 1)
    h = F.group_norm(h, 4, gm.double(), bt.double(), 1e-5)
    ref_y = F.silu(F.group_norm(h, 4, gm.double(), bt.double(), 1e-5))
    ref_z = O.dwconv1d(x1, w1.squeeze(1), b1, 3, 512 + 3)
    assert O.max_rel_err(y.cpu(), ref_y) <= 1e-2
    assert O.max_rel_err(z.cpu(), ref_z) <= 1e-2

    # training: gradients of every input through the ops' autograd formulas
    torch._dynamo.reset()
    compiled = torch.compile(block, backend="aot_eager", fullgraph=True)
    leaves = [t.clone().requires_grad_(True) for t in dev_args]
    y, z = compiled(*leaves)
    gy = torch.randn(y.shape, generator=g).to(dt)
    gz = torch.randn(z.shape, generator=g).to(dt)
    grads = torch.autograd.grad((y, z), leaves, (gy.to(dev), gz.to(dev)))
    ref_leaves = [t.double().requires_grad_(True) for t in (x, w3, b3, gm, bt, x1, w1, b1)]

    def block64(x, w3, b3, gm, bt, x1, w1, b1):
        h = F.group_norm(F.conv3d(x, w3, b3, 1, 1), 4, gm, bt, 1e-5)
        return (F.silu(F.group_norm(h, 4, gm, bt, 1e-5)),
                att.miopen_fallback._original_conv1d(x1, w1, b1, 1, 3, 1, 32))
    ry, rz = block64(*ref_leaves)
    ref_grads = torch.autograd.grad((ry, rz), ref_leaves, (gy.double(), gz.double()))
    for i, (a, r) in enumerate(zip(grads, ref_grads)):
        err = O.max_rel_err(a.cpu(), r)
        assert err <= 1e-2, f"grad {i}: {err:.3g}"


def test_two_streams_do_not_share_scratch(dev):
    """A conv3d (packed weights + split-K partials in scratch) and a multi-slice GroupNorm
    (slot table) of different shapes, issued interleaved on two streams: each stream gets
    its own workspaces and every output matches the oracle."""
    att = _att()
    nat = att._native
    gen = torch.Generator().manual_seed(55)
    shapes = [((1, 64, 64, 64, 16), (1, 32, 8, 16, 16)), ((1, 32, 128, 128, 4), (1, 64, 4, 8, 8))]
    jobs = []
    for (gn_shape, conv_shape) in shapes:
        xg = torch.randn(gn_shape, generator=gen).to(torch.bfloat16)
        gm = (1 + 0.1 * torch.randn(gn_shape[1], generator=gen)).to(torch.bfloat16)
        bt = (0.1 * torch.randn(gn_shape[1], generator=gen)).to(torch.bfloat16)
        xc = torch.randn(conv_shape, generator=gen).to(torch.bfloat16)
        wc = (torch.randn(conv_shape[1], conv_shape[1], 3, 3, 3, generator=gen)
              * (2.0 / (conv_shape[1] * 27)) ** 0.5).to(torch.bfloat16)
        jobs.append((xg, gm, bt, xc, wc))
    refs = [(O.group_norm(xg, 32, gm, bt, 1e-5), O.conv3d(xc, wc, None, 1, 1, 1))
            for xg, gm, bt, xc, wc in jobs]
    names = nat.variants(nat.OP_GROUP_NORM)
    gn_v = names.index("res_nt256_v8")
    streams = [torch.cuda.Stream(dev), torch.cuda.Stream(dev)]
    dev_jobs = [[t.to(dev) for t in job] for job in jobs]

    def mfma_variant(xc, wc):  # an implicit-GEMM tile taking the shape (it packs weights in scratch)
        for vi, name in enumerate(nat.variants(nat.OP_CONV)):
            if name.startswith("h_"):
                try:
                    nat.conv3d(xc, wc, None, 1, 1, 1, variant=vi)
                    return vi
                except nat.Unsupported:
                    continue
        raise AssertionError("no MFMA tile takes the shape")
    conv_v = [mfma_variant(job[3], job[4]) for job in dev_jobs]
    torch.cuda.synchronize()
    outs = [[], []]
    for rep in range(4):
        for k, (s, (xg, gm, bt, xc, wc)) in enumerate(zip(streams, dev_jobs)):
            with torch.cuda.stream(s):
                outs[k].append((nat.group_norm(xg, 32, gm, bt, 1e-5, variant=gn_v),
                                nat.conv3d(xc, wc, None, 1, 1, 1, variant=conv_v[k])))
    torch.cuda.synchronize()
    keys = nat.workspace_keys()
    handles = {s.cuda_stream for s in streams}
    for purpose in ("group_norm", "conv"):
        assert {h for (_, h, p) in keys if p == purpose} >= handles, keys
    for k in range(2):
        for y_gn, y_conv in outs[k]:
            assert O.max_rel_err(y_gn.cpu(), refs[k][0]) <= 1e-2
            assert O.max_rel_err(y_conv.cpu(), refs[k][1]) <= 1e-2
    assert not nat.group_norm_barrier_error(dev)
