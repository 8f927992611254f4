"""GPU parity of the channels-last depthwise conv1d kernels (C ABI atk_dwconv1d_cl_fwd,
atk_dwconv1d_cl_bwd_weight, atk_causal_conv1d_cl_bwd through the ctypes binding) against the
float64 oracle:

* the reference's BLH depthwise conv1d (`conv1d_forward(..., is_bhl=False)`, weight [K, C]),
  forward and autograd backward;
* causal_conv1d_fn on channel-last x (x.stride(1) == 1), with initial / final states and
  seq_idx, forward and backward, at the reference test's shapes and layouts
  (src/causal-conv1d-amd/tests/test_causal_conv1d.py:16-140, 215-270: x a slice of a wider
  (batch, seqlen, 4096 + dim + 64) tensor, fp32 weights);
* the (B, C, L) causal autograd path with SiLU.

Bars: fp32 max-abs-rel <= 1e-5, fp16/bf16 <= 1e-2 against the float64 oracle, and the
reference test's own allclose tolerances."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
BAR = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 1e-2}
# the reference test's tolerances (test_causal_conv1d.py:41-45)
RTOL_ATOL = {torch.float32: (3e-4, 1e-3), torch.float16: (3e-3, 5e-3), torch.bfloat16: (1e-2, 5e-2)}


def _close(y, ref64, dtype, what):
    ref = torch.from_numpy(np.ascontiguousarray(ref64))
    err = O.max_rel_err(y, ref64)
    assert err <= BAR[dtype], f"{what}: max_rel_err {err:.3g} > {BAR[dtype]}"
    rtol, atol = RTOL_ATOL[dtype]
    assert torch.allclose(y.detach().double().cpu(), ref, rtol=rtol, atol=atol), what


def _grad_close(g, ref64, what, bar=1e-5):
    """Weight / bias gradients come back in fp32 from fp32 accumulation: held to 1e-5 of the
    largest entry (the reference test allows rtol = atol = 1e-3)."""
    err = O.max_rel_err(g.float(), ref64)
    assert err <= bar, f"{what}: max_rel_err {err:.3g} > {bar}"


# ---------------------------------------------------------------------------
# BLH depthwise conv1d (conv1d_forward / DepthwiseConv1dFn with is_bhl=False)
# ---------------------------------------------------------------------------
BLH_CASES = [
    # (B, L, D, K, padding)
    (2, 37, 64, 3, 1),
    (2, 100, 128, 5, 2),
    (1, 1, 64, 3, 1),
    (2, 333, 256, 7, 3),
    (3, 64, 72, 1, 0),
    (2, 50, 64, 3, 0),      # 'valid'
    (1, 2048, 512, 3, 1),
]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", BLH_CASES)
def test_blh_forward_matches_oracle(case, dtype):
    from amd_tuned_torch import depthwise_conv1d_ops as ops
    B, L, D, K, pad = case
    g = torch.Generator().manual_seed(B * L + D + K)
    u = torch.randn(B, L, D, generator=g).to(dtype)
    w = (torch.randn(K, D, generator=g) / K ** 0.5).to(dtype)
    b = (torch.randn(D, generator=g) * 0.3).to(dtype)
    y = ops.conv1d_forward(u.cuda(), w.cuda(), b.cuda(), pad, False)
    l_out = L + 2 * pad - K + 1
    assert tuple(y.shape) == (B, l_out, D) and y.is_contiguous()
    ref = O.dwconv1d(u.transpose(1, 2), w.t(), b, pad, l_out).transpose(0, 2, 1)
    _close(y, ref, dtype, "blh forward")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", [(2, 37, 64, 3, 1), (2, 100, 128, 5, 2), (1, 700, 256, 3, 1), (2, 50, 64, 3, 0)])
def test_blh_backward_matches_oracle(case, dtype):
    from amd_tuned_torch import depthwise_conv1d_ops as ops
    B, L, D, K, pad = case
    g = torch.Generator().manual_seed(11 + L)
    u = torch.randn(B, L, D, generator=g).to(dtype).cuda().requires_grad_()
    w = (torch.randn(K, D, generator=g) / K ** 0.5).to(dtype).cuda().requires_grad_()
    b = (torch.randn(D, generator=g) * 0.3).to(dtype).cuda().requires_grad_()
    y = ops.DepthwiseConv1dFn.apply(u, w, b, pad, False)
    dy = torch.randn(y.shape, generator=g).to(dtype)
    y.backward(dy.cuda())
    dx, dw, db = O.dwconv1d_bwd(u.detach().transpose(1, 2), w.detach().t(), dy.transpose(1, 2), pad)
    _close(u.grad, dx.transpose(0, 2, 1), dtype, "blh du")
    assert w.grad.shape == w.shape and w.grad.dtype == dtype
    _grad_close(w.grad, dw.T, "blh dweight", 1e-5 if dtype == torch.float32 else 1e-2)
    _grad_close(b.grad, db, "blh dbias", 1e-5 if dtype == torch.float32 else 1e-2)


# (B, L, D, K, pad_left, L_out): symmetric, 'valid', pad beyond K-1, one-sided, L = 1, and a
# long row spanning several per-thread runs
CL_BWD_FUSED = [
    (2, 37, 64, 3, 1, 37),
    (2, 50, 64, 3, 0, 48),
    (3, 41, 128, 4, 3, 41),      # the causal form
    (2, 29, 64, 2, 2, 31),       # pad_left = K: output longer than the input
    (2, 33, 64, 3, 1, 32),       # one-sided: pad_left 1, pad_right 0
    (1, 1, 64, 3, 1, 1),
    (2, 2500, 256, 3, 1, 2500),
]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", CL_BWD_FUSED, ids=lambda c: "_".join(map(str, c)))
def test_blh_fused_backward_matches_oracle(case, dtype):
    """atk_dwconv1d_cl_bwd (dx, dw, db in one pass) against the float64 oracle, on views: x a
    channel slice of a wider tensor, dy dense; weight (D, K) as the transposed [K, D] view."""
    from amd_tuned_torch import _native as nat
    B, L, D, K, pad, l_out = case
    g = torch.Generator().manual_seed(B * L + D + K + pad)
    big = torch.randn(B, L, D + 64, generator=g).to(dtype)
    x = big.cuda()[:, :, 32:32 + D]
    w = (torch.randn(K, D, generator=g) / K ** 0.5).to(dtype)
    dy = torch.randn(B, l_out, D, generator=g).to(dtype)
    dx, dw, db = nat.dwconv1d_cl_bwd(x, dy.cuda(), w.cuda().t(), pad)
    torch.cuda.synchronize()
    rdx, rdw, rdb = O.dwconv1d_bwd(x.cpu().transpose(1, 2), w.t(), dy.transpose(1, 2), pad)
    _close(dx, rdx.transpose(0, 2, 1), dtype, "fused dx")
    _grad_close(dw, rdw, "fused dw", 1e-5 if dtype == torch.float32 else 1e-2)
    _grad_close(db, rdb, "fused db", 1e-5 if dtype == torch.float32 else 1e-2)
    dx2, dw2, db2 = nat.dwconv1d_cl_bwd(x, dy.cuda(), w.cuda().t(), pad)
    assert torch.equal(dx, dx2) and torch.equal(dw, dw2) and torch.equal(db, db2), "not deterministic"


# ---------------------------------------------------------------------------
# causal_conv1d_fn, channel-last
# ---------------------------------------------------------------------------
def _cl_inputs(batch, dim, seqlen, width, dtype, seed, has_bias=True, has_init=False):
    g = torch.Generator(device="cuda").manual_seed(seed)
    big = torch.randn(batch, seqlen, 4096 + dim + 64, device="cuda", generator=g).to(dtype)
    x = big[:, :, 4096:4096 + dim].transpose(1, 2)
    w = torch.randn(dim, width, device="cuda", generator=g)
    b = torch.randn(dim, device="cuda", generator=g) if has_bias else None
    init = torch.randn(batch, width - 1, dim, device="cuda", generator=g).to(dtype).transpose(1, 2) \
        if has_init else None
    return x, w, b, init


# the reference test's seqlens (test_causal_conv1d.py:30-32) at dim 64; a subset at 4096 + 32
CL_FWD = [(64, s) for s in (1, 2, 8, 16, 32, 64, 128, 129, 130, 151, 256, 372, 512, 784, 1024, 1134, 2048, 4096)] + \
    [(4096 + 32, s) for s in (1, 129, 1134)]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("width", [2, 3, 4])
@pytest.mark.parametrize("dim,seqlen", CL_FWD)
def test_causal_channel_last_forward_with_states(dim, seqlen, width, dtype):
    from amd_tuned_torch.causal_conv1d import causal_conv1d_fn
    for silu, has_init, final in ((False, False, False), (True, True, True), (False, True, True), (True, False, True)):
        x, w, b, init = _cl_inputs(2, dim, seqlen, width, dtype, seqlen + width + dim, True, has_init)
        assert x.stride(1) == 1 and x.stride(2) > 1
        out = causal_conv1d_fn(x, w, b, initial_states=init, return_final_states=final,
                               activation="silu" if silu else None)
        y, fin = (out if final else (out, None))
        assert y.stride() == torch.empty_like(x).stride()
        ry, rfin = O.causal_conv1d_states(x, w, b, initial_states=init, silu=silu)
        _close(y, ry, dtype, f"out silu={silu} init={has_init}")
        if final:
            assert fin.shape == (2, dim, width - 1) and fin.stride(1) == 1
            assert torch.equal(fin.double().cpu(), torch.from_numpy(rfin)), "final states are copies of x"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("width", [2, 3, 4])
@pytest.mark.parametrize("seqlen", [1, 8, 129, 372, 1134])
def test_causal_channel_last_backward_with_states(seqlen, width, dtype):
    from amd_tuned_torch.causal_conv1d import causal_conv1d_fn
    dim = 64
    for silu in (False, True):
        x, w, b, init = _cl_inputs(2, dim, seqlen, width, dtype, 3 * seqlen + width, True, True)
        x, w, b, init = (t.detach().requires_grad_() for t in (x, w, b, init))
        y, fin = causal_conv1d_fn(x, w, b, initial_states=init, return_final_states=True,
                                  activation="silu" if silu else None)
        g = torch.Generator(device="cuda").manual_seed(5 + seqlen)
        dy = torch.randn(y.shape, device="cuda", generator=g).to(dtype)
        dfin = torch.randn(fin.shape, device="cuda", generator=g).to(dtype)
        torch.autograd.backward([y, fin], [dy, dfin])
        dx, dw, db, dinit = O.causal_conv1d_states_bwd(x.detach(), w.detach(), b.detach(), dy,
                                                       initial_states=init.detach(), dfinal=dfin, silu=silu)
        assert init.grad.stride(1) == 1  # (x is a non-dense slice: autograd lays its grad out anew)
        _close(x.grad, dx, dtype, f"dx silu={silu}")
        _close(init.grad, dinit, dtype, f"dinitial_states silu={silu}")
        assert w.grad.dtype == torch.float32
        _grad_close(w.grad, dw, f"dweight silu={silu}", 1e-5 if dtype == torch.float32 else 2e-3)
        _grad_close(b.grad, db, f"dbias silu={silu}", 1e-5 if dtype == torch.float32 else 2e-3)
        rtolw = atolw = 1e-3
        assert torch.allclose(w.grad.double().cpu(), torch.from_numpy(dw), rtol=rtolw, atol=atolw)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("width", [2, 3, 4])
@pytest.mark.parametrize("seqlen", [8, 129, 372, 1024, 2048])
def test_causal_channel_last_seq_idx(seqlen, width, dtype):
    """Sequences packed along the length, split as the reference test splits them
    (test_causal_conv1d.py:233-245); forward and backward."""
    from amd_tuned_torch.causal_conv1d import causal_conv1d_fn
    rng = np.random.default_rng(seqlen + width)
    batch, dim = 3, 64
    seq = []
    for _ in range(batch):
        ns = int(rng.integers(1, 5))
        eos = np.sort(rng.permutation(seqlen - 1)[:ns])
        lens = np.diff(np.concatenate([[-1], eos, [seqlen - 1]]))
        seq.append(np.concatenate([np.full(int(s), i, dtype=np.int32) for i, s in enumerate(lens) if s > 0]))
    seq_idx = torch.from_numpy(np.stack(seq)).cuda()
    for silu in (False, True):
        x, w, b, _ = _cl_inputs(batch, dim, seqlen, width, dtype, seqlen * width, True)
        x, w, b = (t.detach().requires_grad_() for t in (x, w, b))
        y = causal_conv1d_fn(x, w, b, seq_idx=seq_idx, activation="silu" if silu else None)
        ry, _ = O.causal_conv1d_states(x.detach(), w.detach(), b.detach(), seq_idx=seq_idx, silu=silu)
        _close(y, ry, dtype, f"seq_idx out silu={silu}")
        dy = torch.randn(y.shape, device="cuda", generator=torch.Generator(device="cuda").manual_seed(seqlen)).to(dtype)
        y.backward(dy)
        dx, dw, db, _ = O.causal_conv1d_states_bwd(x.detach(), w.detach(), b.detach(), dy, seq_idx=seq_idx,
                                                   silu=silu)
        _close(x.grad, dx, dtype, f"seq_idx dx silu={silu}")
        _grad_close(w.grad, dw, "seq_idx dweight", 1e-5 if dtype == torch.float32 else 2e-3)
        _grad_close(b.grad, db, "seq_idx dbias", 1e-5 if dtype == torch.float32 else 2e-3)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("silu", [False, True])
@pytest.mark.parametrize("L,K", [(256, 4), (4096, 4), (1024, 2), (512, 3), (300, 4)])
def test_causal_bcl_autograd(dtype, silu, L, K):
    """The (B, C, L) layout through causal_conv1d_fn's backward (fp32 weights): the fused
    kernel (L a multiple of 16 bytes) and the composition it falls back to (L = 300)."""
    from amd_tuned_torch.causal_conv1d import causal_conv1d_fn
    g = torch.Generator().manual_seed(3 + L + K)
    B, D = 2, 64
    x = torch.randn(B, D, L, generator=g).to(dtype).cuda().requires_grad_()
    w = torch.randn(D, K, generator=g).cuda().requires_grad_()
    b = torch.randn(D, generator=g).cuda().requires_grad_()
    y = causal_conv1d_fn(x, w, b, activation="silu" if silu else None)
    dy = torch.randn(y.shape, generator=g).to(dtype).cuda()
    y.backward(dy)
    # fp32 weights and bias are used unrounded (the reference dispatches the weight type
    # separately): the oracle gets them as given
    wq, bq = w.detach(), b.detach()
    ry, _ = O.causal_conv1d_states(x.detach(), wq, bq, silu=silu)
    _close(y, ry, dtype, "bcl out")
    dx, dw, db, _ = O.causal_conv1d_states_bwd(x.detach(), wq, bq, dy, silu=silu)
    _close(x.grad, dx, dtype, "bcl dx")
    _grad_close(w.grad, dw, "bcl dweight", 1e-5 if dtype == torch.float32 else 2e-3)
    _grad_close(b.grad, db, "bcl dbias", 1e-5 if dtype == torch.float32 else 2e-3)


# channels checked against the float64 oracle in the full-size tests: first, last, a power of
# two and two odd ones, over all 16 batch rows
_SAMPLED_CHANNELS = [0, 1, 511, 1024, 2047]


def test_causal_channel_last_full_size_matches_bcl_kernel():
    """C2's shape (16, 2048, 8192) bf16 in the channel-last layout, K = 4, against the
    parity-tested (B, C, L) kernel on the same values, and its backward against the
    (B, C, L) backward composition."""
    from amd_tuned_torch import _native
    from amd_tuned_torch.causal_conv1d import causal_conv1d_fn
    g = torch.Generator(device="cuda").manual_seed(0)
    B, D, L, K = 16, 2048, 8192, 4
    x_cl = torch.randn(B, L, D, device="cuda", generator=g).to(torch.bfloat16).transpose(1, 2)
    w = (torch.randn(D, K, device="cuda", generator=g) / 2).to(torch.bfloat16)
    b = (torch.randn(D, device="cuda", generator=g) * 0.1).to(torch.bfloat16)
    y = causal_conv1d_fn(x_cl, w, b)
    y_ref = _native.dwconv1d(x_cl.contiguous(), w, b, K - 1, L)
    assert O.max_rel_err(y.float(), y_ref.float()) <= 1e-2
    assert (y.contiguous() == y_ref).float().mean().item() > 0.99
    # backward: dx, dw, db against the (B, C, L) composition
    xr = x_cl.detach().requires_grad_()
    wr = w.detach().float().requires_grad_()
    br = b.detach().float().requires_grad_()
    out = causal_conv1d_fn(xr, wr, br)
    dy = torch.randn(B, L, D, device="cuda", generator=g).to(torch.bfloat16).transpose(1, 2)
    out.backward(dy)
    dyc = dy.contiguous()
    dx_ref = _native.dwconv1d(dyc, w.flip(-1), None, 0, L)
    dw_ref, db_ref = _native.dwconv1d_bwd_weight(x_cl.contiguous(), dyc, K, K - 1)
    assert O.max_rel_err(xr.grad.float(), dx_ref.float()) <= 1e-2
    assert O.max_rel_err(wr.grad, dw_ref) <= 1e-4
    assert O.max_rel_err(br.grad, db_ref) <= 1e-4
    # and against the float64 oracle on sampled channels (channels are independent: a few
    # whole channels over every batch row pin forward, dx, dw and db exactly)
    cs = torch.tensor(_SAMPLED_CHANNELS, device="cuda")
    xs = x_cl.index_select(1, cs).cpu()
    dys = dy.index_select(1, cs).cpu()
    ws, bs = wr.detach().index_select(0, cs).cpu(), br.detach().index_select(0, cs).cpu()
    _close(y.index_select(1, cs), O.dwconv1d(xs, ws, bs, K - 1, L), torch.bfloat16, "full-size forward")
    dxo, dwo, dbo = O.dwconv1d_bwd(xs, ws, dys, K - 1)
    _close(xr.grad.index_select(1, cs), dxo, torch.bfloat16, "full-size dx")
    _grad_close(wr.grad.index_select(0, cs), dwo, "full-size dweight", 1e-5)
    _grad_close(br.grad.index_select(0, cs), dbo, "full-size dbias", 1e-5)
    del x_cl, y, y_ref, xr, out, dy, dyc, dx_ref
    torch.cuda.empty_cache()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("K,pad", [(4, 3), (3, 1), (5, 0)])
def test_fconv1d_on_channel_last_input_takes_the_channels_last_kernel(K, pad, dtype):
    """Patched F.conv1d on a channel-last x (sliced like the reference test's inputs): the
    depthwise call runs the channels-last kernel (output returned channel-last, like
    causal_conv1d_fn's) and its backward; values and gradients match the oracle."""
    import torch.nn.functional as F
    import amd_tuned_torch  # noqa: F401
    B, D, L = 2, 64, 300
    g = torch.Generator(device="cuda").manual_seed(K * 10 + pad)
    big = torch.randn(B, L, D + 64, device="cuda", generator=g).to(dtype)
    x = big[:, :, 32:32 + D].transpose(1, 2)
    w = (torch.randn(D, 1, K, device="cuda", generator=g) / K ** 0.5).to(dtype)
    b = (torch.randn(D, device="cuda", generator=g) * 0.3).to(dtype)
    l_out = L + 2 * pad - K + 1
    y = F.conv1d(x, w, b, padding=pad, groups=D)
    assert y.shape == (B, D, l_out) and y.stride(1) == 1, "not the channels-last route"
    _close(y, O.dwconv1d(x, w, b, pad, l_out), dtype, "F.conv1d channel-last forward")
    xg, wg, bg = (t.detach().requires_grad_() for t in (x, w, b))
    yg = F.conv1d(xg, wg, bg, padding=pad, groups=D)
    dy = torch.randn(yg.shape, device="cuda", generator=g).to(dtype)
    yg.backward(dy)
    dx, dw, db = O.dwconv1d_bwd(x, w, dy, pad)
    _close(xg.grad, dx, dtype, "F.conv1d channel-last dx")
    _grad_close(wg.grad.reshape(D, K), dw, "dweight", 1e-5 if dtype == torch.float32 else 1e-2)
    _grad_close(bg.grad, db, "dbias", 1e-5 if dtype == torch.float32 else 1e-2)


def test_causal_bcl_fused_backward_full_size():
    """Config 2's shape (16, 2048, 8192) bf16, K = 4: the fused (B, C, L) backward against the
    composition of parity-tested kernels (forward kernel on the flipped weights for dx, the
    weight-gradient kernel for dw / db)."""
    from amd_tuned_torch import _native
    g = torch.Generator(device="cuda").manual_seed(1)
    B, D, L, K = 16, 2048, 8192, 4
    x = torch.randn(B, D, L, device="cuda", generator=g).to(torch.bfloat16)
    dy = torch.randn(B, D, L, device="cuda", generator=g).to(torch.bfloat16)
    w = (torch.randn(D, K, device="cuda", generator=g) / 2).to(torch.bfloat16)
    dx, dw, db = _native.causal_conv1d_bwd(x, dy, w, None, silu=False)
    dx_ref = _native.dwconv1d(dy, w.flip(-1), None, 0, L)
    dw_ref, db_ref = _native.dwconv1d_bwd_weight(x, dy, K, K - 1)
    assert O.max_rel_err(dx.float(), dx_ref.float()) <= 1e-2
    assert (dx == dx_ref).float().mean().item() > 0.99
    assert O.max_rel_err(dw, dw_ref) <= 1e-4 and O.max_rel_err(db, db_ref) <= 1e-4
    # against the float64 oracle on sampled whole channels (every batch row)
    cs = torch.tensor(_SAMPLED_CHANNELS, device="cuda")
    dxo, dwo, dbo = O.dwconv1d_bwd(x.index_select(1, cs).cpu(), w.index_select(0, cs).cpu(),
                                   dy.index_select(1, cs).cpu(), K - 1)
    _close(dx.index_select(1, cs), dxo, torch.bfloat16, "full-size fused dx")
    _grad_close(dw.index_select(0, cs), dwo, "full-size fused dweight", 1e-5)
    _grad_close(db.index_select(0, cs), dbo, "full-size fused dbias", 1e-5)
    del x, dy, dx, dx_ref
    torch.cuda.empty_cache()


# The (B, C, L) causal path and the decode step use fp32 weights unrounded, as the
# reference does (causal_conv1d.cpp:139-141, 437).  A cancellation makes rounding visible:
# with w = (1 + 2^-12, -1) on all-ones input, y = 2^-12 exactly (representable in fp16 and
# bf16), while weights rounded to fp16 / bf16 (1 + 2^-12 -> 1) would give 0.
EPS_W = 2.0 ** -12


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("L", [64, 300])
def test_causal_bcl_fp32_weights_are_not_rounded(dtype, L):
    from amd_tuned_torch.causal_conv1d import causal_conv1d_fn
    B, D, K = 2, 8, 2
    x = torch.ones(B, D, L, dtype=dtype, device="cuda", requires_grad=True)
    w = torch.tensor([1.0 + EPS_W, -1.0], dtype=torch.float32).repeat(D, 1).cuda().requires_grad_()
    y = causal_conv1d_fn(x, w)
    ry, _ = O.causal_conv1d_states(x.detach(), w.detach())
    assert ry[0, 0, 1] == EPS_W and ry[0, 0, 0] == -1.0
    assert torch.equal(y.detach().double().cpu(), torch.from_numpy(ry)), "forward used rounded weights"
    # backward: dx of the same cancellation (L = 300 takes the composed fallback)
    dy = torch.ones(B, D, L, dtype=dtype, device="cuda")
    y.backward(dy)
    rdx, rdw, _, _ = O.causal_conv1d_states_bwd(x.detach(), w.detach(), None, dy)
    assert torch.equal(x.grad.double().cpu(), torch.from_numpy(rdx)), "backward used rounded weights"
    _grad_close(w.grad, rdw, "dweight")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_causal_conv1d_update_fp32_weights_are_not_rounded(dtype):
    from amd_tuned_torch import causal_conv1d as cc
    B, D, W = 3, 16, 2
    x = torch.ones(B, D, dtype=dtype, device="cuda")
    st = torch.ones(B, D, W, dtype=dtype, device="cuda")
    w = torch.tensor([1.0 + EPS_W, -1.0], dtype=torch.float32).repeat(D, 1).cuda()
    b = torch.zeros(D, dtype=torch.float32, device="cuda")
    y = cc.causal_conv1d_update(x, st, w, b)
    assert torch.all(y.double().cpu() == EPS_W), "decode step used rounded weights"
    # and on random data it matches the float64 oracle with the fp32 weights as given
    g = torch.Generator().manual_seed(99)
    x2 = torch.randn(B, D, generator=g).to(dtype)
    st2 = torch.randn(B, D, 4, generator=g).to(dtype)
    w2 = torch.randn(D, 4, generator=g) * 0.5
    b2 = 0.1 * torch.randn(D, generator=g)
    sd = st2.cuda()
    y2 = cc.causal_conv1d_update(x2.cuda(), sd, w2.cuda(), b2.cuda(), activation="silu")
    ry, rs = O.causal_conv1d_update(x2, st2, w2, b2, True)
    assert O.max_rel_err(y2.cpu(), ry) <= BAR[dtype]
    assert torch.equal(sd.cpu().double(), torch.from_numpy(rs))
