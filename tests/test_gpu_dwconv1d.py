"""GPU parity of the depthwise conv1d kernel (C ABI atk_dwconv1d_fwd through the ctypes
binding) against the float64 oracle.  Bars: fp32 max-abs-rel <= 1e-5, fp16/bf16 <= 1e-2
(fp32 accumulation)."""
from __future__ import annotations

import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
BAR = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 1e-2}


def _native():
    from amd_tuned_torch import _native
    return _native


def _inputs(N, C, L, K, dtype, seed=0, bias=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(N, C, L, generator=g)
    w = torch.randn(C, K, generator=g) * (1.0 / K) ** 0.5
    b = torch.randn(C, generator=g) * 0.1 ** 0.5 if bias else None
    return x.to(dtype), w.to(dtype), (b.to(dtype) if b is not None else None)


def _check(y, x, w, b, pad, l_out, silu=False):
    ref = O.dwconv1d(x, w, b, pad, l_out, silu=silu)
    assert tuple(y.shape) == ref.shape
    err = O.max_rel_err(y, ref)
    assert err <= BAR[y.dtype], f"max_rel_err {err:.3g} > {BAR[y.dtype]}"
    return err


CASES = [
    # (N, C, L, K, pad_left, l_out)
    (2, 3, 37, 3, 1, 37),        # symmetric
    (2, 3, 37, 4, 3, 40),        # causal, stock output shape (rows not 16B aligned)
    (2, 3, 37, 4, 3, 37),        # causal, truncated to L
    (2, 5, 64, 2, 1, 65),        # causal K=2
    (1, 4, 100, 5, 2, 100),
    (2, 2, 50, 7, 3, 50),        # generic-K path
    (1, 3, 40, 31, 15, 40),      # wide kernel
    (1, 2, 30, 3, 0, 28),        # 'valid' (L_out < L)
    (1, 2, 10, 3, 5, 18),        # padding wider than the kernel
    (3, 7, 1, 3, 1, 1),          # L = 1
    (2, 16, 8, 1, 0, 8),         # K = 1
    (1, 8, 4096, 4, 3, 4099),    # long rows, stock causal
    (4, 64, 333, 3, 1, 333),     # many short rows per tile
    # rows longer than a wave's 64 vectors: the cross-lane kernel's in-row path
    (2, 4, 2500, 4, 3, 2503),    # causal, stock shape (row starts at every alignment)
    (1, 6, 2048, 3, 1, 2048),    # symmetric, aligned rows
    (1, 5, 1100, 2, 1, 1101),    # K = 2
    (1, 3, 2000, 5, 2, 2000),    # K = 5
]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_dwconv1d_all_variants(dev, case, dtype):
    N, C, L, K, pad, l_out = case
    nat = _native()
    x, w, b = _inputs(N, C, L, K, dtype, seed=sum(case))
    xd, wd, bd = x.to(dev), w.to(dev), b.to(dev)
    ran = 0
    for vi, name in enumerate(nat.variants(nat.OP_DWCONV1D)):
        try:
            y = nat.dwconv1d(xd, wd, bd, pad, l_out, variant=vi)
        except nat.Unsupported:
            # a tile variant may decline (e.g. its LDS window exceeds 64 KB for fp32);
            # the direct kernel is the one that must take every shape
            assert name != "direct", "the direct variant must accept every shape"
            continue
        torch.cuda.synchronize()
        _check(y.cpu(), x, w, b, pad, l_out)
        ran += 1
    assert ran >= 2


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_dwconv1d_no_bias_and_silu(dev, dtype):
    nat = _native()
    x, w, _ = _inputs(2, 6, 123, 4, dtype, seed=7, bias=False)
    y = nat.dwconv1d(x.to(dev), w.to(dev), None, 3, 126)
    _check(y.cpu(), x, w, None, 3, 126)
    x, w, b = _inputs(2, 6, 123, 4, dtype, seed=8)
    y = nat.dwconv1d(x.to(dev), w.to(dev), b.to(dev), 3, 123, silu=True)
    _check(y.cpu(), x, w, b, 3, 123, silu=True)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_dwconv1d_misaligned_pointers(dev, dtype):
    """x and y views whose data pointers are not 16-byte aligned."""
    nat = _native()
    N, C, L, K = 2, 5, 77, 3
    x, w, b = _inputs(N, C, L, K, dtype, seed=3)
    xb = torch.zeros(N * C * L + 3, dtype=dtype)
    xb[1:1 + N * C * L] = x.flatten()
    xv = xb.to(dev)[1:1 + N * C * L].view(N, C, L)
    for l_out, pad in ((L, 1), (L + 2, 2)):
        ob = torch.full((N * C * l_out + 5,), float("nan"), dtype=dtype, device=dev)
        yv = ob[3:3 + N * C * l_out].view(N, C, l_out)
        for vi, name in enumerate(nat.variants(nat.OP_DWCONV1D)):
            try:
                nat.dwconv1d(xv, w.to(dev), b.to(dev), pad, l_out, variant=vi, out=yv)
            except nat.Unsupported:
                assert name != "direct", "the direct variant must accept every shape"
                continue
            torch.cuda.synchronize()
            _check(yv.cpu(), x, w, b, pad, l_out)
            # the guard elements around the output view are untouched
            assert torch.isnan(ob[:3].float()).all() and torch.isnan(ob[3 + N * C * l_out:].float()).all()


def test_dwconv1d_empty_batch(dev):
    nat = _native()
    x = torch.zeros(0, 4, 16, device=dev)
    y = nat.dwconv1d(x, torch.zeros(4, 3, device=dev), None, 1, 16)
    assert y.shape == (0, 4, 16)


def test_dwconv1d_rejects_bad_args(dev):
    nat = _native()
    x = torch.zeros(1, 4, 16, device=dev)
    with pytest.raises(RuntimeError):
        nat.dwconv1d(x, torch.zeros(5, 3, device=dev), None, 1, 16)       # channel mismatch
    with pytest.raises(nat.Unsupported):
        nat.dwconv1d(x, torch.zeros(4, 65, device=dev), None, 1, 16)      # K > 64
    with pytest.raises(RuntimeError):
        nat.dwconv1d(x, torch.zeros(4, 3, device=dev, dtype=torch.float16), None, 1, 16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("mode", ["causal_stock", "causal_trunc", "symmetric"])
def test_dwconv1d_config2_full_size(dev, dtype, mode):
    """BASELINE config 2 at its full size: N=16, C=2048, L=8192; causal K=4 (stock shape
    and truncated) and symmetric K=3 -- every output checked against the oracle."""
    N, C, L = 16, 2048, 8192
    K, pad, l_out = {"causal_stock": (4, 3, L + 3), "causal_trunc": (4, 3, L),
                     "symmetric": (3, 1, L)}[mode]
    x, w, b = _inputs(N, C, L, K, dtype, seed=1002)
    nat = _native()
    y = nat.dwconv1d(x.to(dev), w.to(dev), b.to(dev), pad, l_out)
    torch.cuda.synchronize()
    _check(y.cpu(), x, w, b, pad, l_out)


# ---------------------------------------------------------------------------
# backward: dx through the forward kernel (reversed weights), dw / db through the
# streaming reduction kernel -- against the float64 oracle
# ---------------------------------------------------------------------------
BWD_BAR_W = {torch.float32: 1e-5, torch.float16: 1e-4, torch.bfloat16: 1e-4}  # fp32 dw/db from exact inputs

BWD_CASES = [
    (2, 3, 37, 3, 1, 37),        # symmetric
    (2, 3, 37, 4, 3, 40),        # causal, stock output shape
    (2, 3, 37, 4, 3, 37),        # causal, truncated
    (2, 5, 64, 2, 1, 65),        # K = 2
    (1, 4, 100, 5, 2, 100),      # K = 5
    (1, 3, 40, 1, 0, 40),        # K = 1
    (1, 2, 30, 3, 0, 28),        # 'valid'
    (1, 8, 4096, 4, 3, 4099),    # long rows
    (2, 4, 2500, 4, 3, 2503),    # long unaligned rows
    (3, 7, 1, 3, 1, 1),          # L = 1
    (1, 3, 64, 3, 4, 70),        # padding above K-1 (fused kernel; the two-kernel form declines dx)
    (2, 2, 32, 3, 0, 30),        # 'valid', aligned rows (fused kernel)
]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("case", BWD_CASES, ids=lambda c: "x".join(map(str, c)))
def test_dwconv1d_backward_native(dev, case, dtype):
    N, C, L, K, pad, l_out = case
    nat = _native()
    x, w, _ = _inputs(N, C, L, K, dtype, seed=sum(case) + 5)
    dy = torch.randn(N, C, l_out, generator=torch.Generator().manual_seed(sum(case))).to(dtype)
    dx, dw, db = nat.dwconv1d_backward(dy.to(dev), x.to(dev), w.to(dev), pad, (True, True, True))
    torch.cuda.synchronize()
    rdx, rdw, rdb = O.dwconv1d_bwd(x, w, dy, pad)
    assert dx.dtype == dtype and dw.dtype == torch.float32 and db.dtype == torch.float32
    assert O.max_rel_err(dx.cpu(), rdx) <= BAR[dtype]
    assert O.max_rel_err(dw.cpu(), rdw) <= BWD_BAR_W[dtype]
    assert O.max_rel_err(db.cpu(), rdb) <= BWD_BAR_W[dtype]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_dwconv1d_autograd_through_patched_conv1d(dev, dtype):
    """Training path: the patched F.conv1d (causal stock shape and symmetric) with
    requires_grad inputs runs the native forward and backward; gradients match the oracle."""
    import torch.nn.functional as F
    import amd_tuned_torch  # noqa: F401  (installs the patch)
    for K, pad, trunc in ((4, 3, True), (4, 3, False), (3, 1, False)):
        N, C, L = 2, 6, 300
        x, w, b = _inputs(N, C, L, K, dtype, seed=11 + K + pad)
        xd = x.to(dev).requires_grad_(True)
        wd = w.to(dev).unsqueeze(1).requires_grad_(True)
        bd = b.to(dev).requires_grad_(True)
        y = F.conv1d(xd, wd, bd, padding=pad, groups=C)
        if trunc:
            y = y[..., :L]
        dy = torch.randn(y.shape, generator=torch.Generator().manual_seed(K)).to(dtype)
        gx, gw, gb = torch.autograd.grad(y, (xd, wd, bd), dy.to(dev))
        rdx, rdw, rdb = O.dwconv1d_bwd(x, w, dy, pad)
        assert O.max_rel_err(gx.cpu(), rdx) <= BAR[dtype]
        assert O.max_rel_err(gw.cpu().reshape(C, K), rdw) <= BAR[dtype]
        assert O.max_rel_err(gb.cpu(), rdb) <= BAR[dtype]


def test_dwconv1d_backward_config2_full_size(dev):
    """BASELINE config 2 at its full size, bf16 causal with the stock output shape: every
    gradient element checked against the oracle."""
    N, C, L, K, pad = 16, 2048, 8192, 4, 3
    nat = _native()
    x, w, _ = _inputs(N, C, L, K, torch.bfloat16, seed=2002)
    dy = torch.randn(N, C, L + 3, generator=torch.Generator().manual_seed(2003)).to(torch.bfloat16)
    dx, dw, db = nat.dwconv1d_backward(dy.to(dev), x.to(dev), w.to(dev), pad, (True, True, True))
    torch.cuda.synchronize()
    rdx, rdw, rdb = O.dwconv1d_bwd(x, w, dy, pad)
    assert O.max_rel_err(dx.cpu(), rdx) <= BAR[torch.bfloat16]
    assert O.max_rel_err(dw.cpu(), rdw) <= BWD_BAR_W[torch.bfloat16]
    assert O.max_rel_err(db.cpu(), rdb) <= BWD_BAR_W[torch.bfloat16]


# ---------------------------------------------------------------------------
# decode step (atk_causal_conv1d_update)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("W,silu", [(2, False), (3, True), (4, False), (4, True)])
def test_causal_conv1d_update_native(dev, W, silu, dtype):
    from amd_tuned_torch import causal_conv1d as cc
    g = torch.Generator().manual_seed(W + 10 * silu)
    B, D = 5, 300
    x = torch.randn(B, D, generator=g).to(dtype)
    st = torch.randn(B, D, W, generator=g).to(dtype)
    w = (torch.randn(D, W, generator=g) * 0.5).to(dtype)
    b = (0.1 * torch.randn(D, generator=g)).to(dtype)
    sd = st.to(dev)
    y = cc.causal_conv1d_update(x.to(dev), sd, w.to(dev), b.to(dev), activation="silu" if silu else None)
    torch.cuda.synchronize()
    ry, rs = O.causal_conv1d_update(x, st, w, b, silu)
    assert O.max_rel_err(y.cpu(), ry) <= BAR[dtype]
    assert torch.equal(sd.cpu().double(), torch.from_numpy(rs))          # the state is moved, not recomputed
    # the reference interface's torch statement agrees
    sr = st.to(dev)
    yr = cc.causal_conv1d_update_ref(x.to(dev), sr, w.to(dev), b.to(dev), activation="silu" if silu else None)
    assert torch.equal(sr.cpu(), sd.cpu())
    assert O.max_rel_err(yr.cpu(), ry) <= BAR[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_causal_conv1d_update_streaming_equals_forward(dev, dtype):
    """Decoding a sequence step by step from a zero state gives the causal forward kernel's
    output (the same fp32 arithmetic), and ends with the last W inputs as the state."""
    from amd_tuned_torch import causal_conv1d as cc
    B, D, L, W = 3, 64, 40, 4
    x, w, b = _inputs(B, D, L, W, dtype, seed=77)
    xd, wd, bd = x.to(dev), w.to(dev), b.to(dev)
    st = torch.zeros(B, D, W, dtype=dtype, device=dev)
    ys = [cc.causal_conv1d_update(xd[:, :, t].contiguous(), st, wd, bd) for t in range(L)]
    full = cc.causal_conv1d_fn(xd, wd, bd)
    torch.cuda.synchronize()
    assert O.max_rel_err(torch.stack(ys, -1).cpu(), O.dwconv1d(x, w, b, W - 1, L)) <= BAR[dtype]
    assert O.max_rel_err(full.cpu(), O.dwconv1d(x, w, b, W - 1, L)) <= BAR[dtype]
    assert torch.equal(st.cpu(), x[:, :, L - W:])
