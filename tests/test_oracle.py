"""Pins the float64 CPU oracle (oracle/atk_oracle.c) before it is trusted as the GPU
parity checker: the committed golden fixtures (stock torch float64), the reference's
depthwise output-length known answers, stock torch on random shapes, brute-force Python
loops, and identities a plausible mistake (dropped term, wrong sign, off-by-one index,
transposed operand) would break."""
from __future__ import annotations

import itertools
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden.npz")


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


# ---------------------------------------------------------------------------
# golden fixtures
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("name", ["dw_sym", "dw_causal", "dw_valid", "dw_widepad"])
def test_dwconv1d_matches_golden(golden, name):
    N, C, L, K, p = golden[f"{name}_meta"].tolist()
    y = O.dwconv1d(golden[f"{name}_x"], golden[f"{name}_w"], golden[f"{name}_b"], p,
                   L + 2 * p - K + 1)
    np.testing.assert_allclose(y, golden[f"{name}_y"], rtol=0, atol=1e-12)


def test_group_norm_matches_golden(golden):
    y = O.group_norm(golden["gn_x"], 3, golden["gn_g"], golden["gn_b"], 1e-5)
    np.testing.assert_allclose(y, golden["gn_y"], rtol=0, atol=1e-12)
    y = O.group_norm(golden["gn_x"], 3, golden["gn_g"], golden["gn_b"], 1e-5, silu=True)
    np.testing.assert_allclose(y, golden["gn_silu_y"], rtol=0, atol=1e-12)
    y = O.group_norm(golden["gn3_x"], 2, None, None, 1e-6)
    np.testing.assert_allclose(y, golden["gn3_y"], rtol=0, atol=1e-12)


def test_conv_matches_golden(golden):
    y = O.conv2d(golden["c2_x"], golden["c2_w"], golden["c2_b"], (2, 1), (1, 2), (1, 2))
    np.testing.assert_allclose(y, golden["c2_y"], rtol=0, atol=1e-12)
    y = O.conv3d(golden["c3_x"], golden["c3_w"], golden["c3_b"], (1, 2, 1), 1, 1)
    np.testing.assert_allclose(y, golden["c3_y"], rtol=0, atol=1e-12)


def _far(a, b) -> bool:
    return a.shape != b.shape or not np.allclose(a, b, rtol=0, atol=1e-9)


def test_golden_pins_catch_planted_mistakes(golden):
    """Each plausible mistake, planted in a call of the oracle, misses the golden fixture:
    off-by-one padding, a flipped (correlation vs convolution) kernel, a dropped bias, a
    wrong group count, a dropped eps, SiLU applied before the affine, and swapped
    stride/dilation or a transposed weight in conv."""
    m = golden["dw_causal_meta"].tolist()
    N, C, L, K, p = m
    x, w, b, y = (golden[f"dw_causal_{k}"] for k in "xwby")
    lo = L + 2 * p - K + 1
    assert _far(O.dwconv1d(x, w, b, p - 1, lo), y)
    assert _far(O.dwconv1d(x, w[..., ::-1].copy(), b, p, lo), y)
    assert _far(O.dwconv1d(x, w, None, p, lo), y)
    gx, gg, gb = golden["gn_x"], golden["gn_g"], golden["gn_b"]
    assert _far(O.group_norm(gx, 1, gg, gb, 1e-5), golden["gn_y"])
    assert _far(O.group_norm(gx, 3, gg, gb, 0.0), golden["gn_y"])
    assert _far(O.group_norm(gx, 3, gg, gb, 1e-5, silu=True), golden["gn_y"])
    silu_first = O.group_norm(gx, 3, None, None, 1e-5, silu=True) * gg.reshape(1, -1, *([1] * (gx.ndim - 2))) \
        + gb.reshape(1, -1, *([1] * (gx.ndim - 2)))
    assert _far(silu_first, golden["gn_silu_y"])
    assert _far(O.conv2d(golden["c2_x"], golden["c2_w"], golden["c2_b"], (1, 2), (1, 2), (2, 1)), golden["c2_y"])
    c3w = golden["c3_w"]
    assert _far(O.conv3d(golden["c3_x"], np.swapaxes(c3w, 3, 4).copy(), golden["c3_b"], (1, 2, 1), 1, 1),
                golden["c3_y"])


# ---------------------------------------------------------------------------
# known answers of the reference's own tests
# ---------------------------------------------------------------------------
def test_out_len_known_answers():
    """tests/test_depthwise_conv1d_ops.py:64-71 of the reference."""
    assert O.conv1d_out_len(10, 1, 3) == 10
    assert O.conv1d_out_len(10, 0, 3) == 8
    assert O.conv1d_out_len(100, 5, 11) == 100
    x = np.zeros((1, 1, 100))
    assert O.dwconv1d(x, np.ones((1, 11)), None, 5, O.conv1d_out_len(100, 5, 11)).shape == (1, 1, 100)


# ---------------------------------------------------------------------------
# brute force (pure Python loops) on tiny shapes
# ---------------------------------------------------------------------------
def _bf_dw(x, w, b, pad, l_out):
    N, C, L = x.shape
    K = w.shape[-1]
    y = np.zeros((N, C, l_out))
    for n, c, t in itertools.product(range(N), range(C), range(l_out)):
        s = b[c] if b is not None else 0.0
        for j in range(K):
            p = t - pad + j
            if 0 <= p < L:
                s += w[c, j] * x[n, c, p]
        y[n, c, t] = s
    return y


def test_dwconv1d_brute_force():
    rng = np.random.default_rng(0)
    for (N, C, L, K, pad, l_out) in [(1, 2, 7, 3, 1, 7), (2, 1, 5, 4, 3, 8), (1, 2, 6, 4, 3, 6),
                                     (1, 1, 4, 2, 5, 10)]:
        x, w, b = rng.normal(size=(N, C, L)), rng.normal(size=(C, K)), rng.normal(size=C)
        np.testing.assert_allclose(O.dwconv1d(x, w, b, pad, l_out), _bf_dw(x, w, b, pad, l_out),
                                   rtol=0, atol=1e-12)


def _bf_conv3d(x, w, b, s, p, d):
    N, Ci, D, H, W = x.shape
    Co, _, KD, KH, KW = w.shape
    Do, Ho, Wo = ((D + 2 * p[0] - d[0] * (KD - 1) - 1) // s[0] + 1,
                  (H + 2 * p[1] - d[1] * (KH - 1) - 1) // s[1] + 1,
                  (W + 2 * p[2] - d[2] * (KW - 1) - 1) // s[2] + 1)
    y = np.zeros((N, Co, Do, Ho, Wo))
    for n, o, z, h, v in itertools.product(range(N), range(Co), range(Do), range(Ho), range(Wo)):
        acc = b[o]
        for i, a, bb, c in itertools.product(range(Ci), range(KD), range(KH), range(KW)):
            iz, iy, ix = z * s[0] - p[0] + a * d[0], h * s[1] - p[1] + bb * d[1], v * s[2] - p[2] + c * d[2]
            if 0 <= iz < D and 0 <= iy < H and 0 <= ix < W:
                acc += w[o, i, a, bb, c] * x[n, i, iz, iy, ix]
        y[n, o, z, h, v] = acc
    return y


def test_conv3d_brute_force():
    rng = np.random.default_rng(1)
    x, w, b = rng.normal(size=(1, 2, 3, 4, 5)), rng.normal(size=(2, 2, 2, 3, 2)), rng.normal(size=2)
    for s, p, d in [((1, 1, 1), (1, 1, 1), (1, 1, 1)), ((2, 1, 2), (0, 2, 1), (1, 1, 2))]:
        np.testing.assert_allclose(O.conv3d(x, w, b, s, p, d), _bf_conv3d(x, w, b, s, p, d),
                                   rtol=0, atol=1e-12)


def test_conv3d_points_subset_matches_full():
    rng = np.random.default_rng(2)
    x, w, b = rng.normal(size=(2, 3, 4, 5, 6)), rng.normal(size=(4, 3, 3, 3, 3)), rng.normal(size=4)
    full = O.conv3d(x, w, b, 1, 1, 1)
    pts = rng.integers(0, full.size, size=50)
    np.testing.assert_allclose(O.conv3d(x, w, b, 1, 1, 1, points=pts), full.ravel()[pts], atol=1e-12)


def _bf_gn(x, G, gm, bt, eps):
    N, C = x.shape[:2]
    y = np.empty_like(x)
    cpg = C // G
    for n in range(N):
        for g in range(G):
            blk = x[n, g * cpg:(g + 1) * cpg]
            mu = sum(blk.ravel()) / blk.size
            var = sum((v - mu) ** 2 for v in blk.ravel()) / blk.size
            for c in range(g * cpg, (g + 1) * cpg):
                y[n, c] = (x[n, c] - mu) / math.sqrt(var + eps) * gm[c] + bt[c]
    return y


def test_group_norm_brute_force():
    rng = np.random.default_rng(3)
    x, gm, bt = rng.normal(size=(2, 4, 3)), rng.normal(size=4), rng.normal(size=4)
    np.testing.assert_allclose(O.group_norm(x, 2, gm, bt, 1e-5), _bf_gn(x, 2, gm, bt, 1e-5),
                               rtol=0, atol=1e-12)


# ---------------------------------------------------------------------------
# stock torch (float64) on random shapes
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("seed", range(4))
def test_oracle_vs_stock_random(seed):
    g = torch.Generator().manual_seed(seed)
    d = torch.float64
    N, C, L = 2, 5, 23 + seed
    K = 1 + seed * 2
    x, w, b = torch.randn(N, C, L, generator=g, dtype=d), torch.randn(C, 1, K, generator=g, dtype=d), torch.randn(C, generator=g, dtype=d)
    for p in (0, (K - 1) // 2, K - 1):
        ref = F.conv1d(x, w, b, padding=p, groups=C).numpy()
        np.testing.assert_allclose(O.dwconv1d(x, w, b, p, ref.shape[-1]), ref, atol=1e-12)
    xs = torch.randn(3, 8, 5, 3, generator=g, dtype=d) * 3 + 7
    gm, bt = torch.randn(8, generator=g, dtype=d), torch.randn(8, generator=g, dtype=d)
    for G in (1, 2, 8):
        np.testing.assert_allclose(O.group_norm(xs, G, gm, bt, 1e-5),
                                   F.group_norm(xs, G, gm, bt, 1e-5).numpy(), atol=1e-11)
    xc, wc, bc = torch.randn(1, 3, 5, 6, 7, generator=g, dtype=d), torch.randn(4, 3, 3, 3, 3, generator=g, dtype=d), torch.randn(4, generator=g, dtype=d)
    np.testing.assert_allclose(O.conv3d(xc, wc, bc, (1, 1, 2), (1, 0, 1), (1, 2, 1)),
                               F.conv3d(xc, wc, bc, (1, 1, 2), (1, 0, 1), (1, 2, 1)).numpy(), atol=1e-11)


# ---------------------------------------------------------------------------
# identities
# ---------------------------------------------------------------------------
def test_delta_kernels_shift_the_input():
    """A one-hot depthwise kernel at tap j shifts every row by j - pad (zero filled);
    a one-hot conv3d kernel at the centre tap with pad 1 is the identity on its channel."""
    rng = np.random.default_rng(4)
    x = rng.normal(size=(1, 2, 9))
    for j in range(4):
        w = np.zeros((2, 4))
        w[:, j] = 1.0
        y = O.dwconv1d(x, w, None, 3, 12)
        for t in range(12):
            p = t - 3 + j
            np.testing.assert_allclose(y[..., t], x[..., p] if 0 <= p < 9 else 0.0, atol=0)
    xc = rng.normal(size=(1, 3, 4, 5, 6))
    w = np.zeros((3, 3, 3, 3, 3))
    for c in range(3):
        w[c, c, 1, 1, 1] = 1.0
    np.testing.assert_allclose(O.conv3d(xc, w, None, 1, 1, 1), xc, atol=0)


def test_linearity():
    rng = np.random.default_rng(5)
    x1, x2 = rng.normal(size=(1, 2, 3, 4, 5)), rng.normal(size=(1, 2, 3, 4, 5))
    w = rng.normal(size=(3, 2, 3, 3, 3))
    np.testing.assert_allclose(O.conv3d(2 * x1 - 3 * x2, w, None, 1, 1, 1),
                               2 * O.conv3d(x1, w, None, 1, 1, 1) - 3 * O.conv3d(x2, w, None, 1, 1, 1),
                               atol=1e-10)


def test_group_norm_invariants():
    """Without affine: each group has mean 0 and variance var/(var+eps); the output is
    invariant to a per-group shift and positive scale (up to the eps term)."""
    rng = np.random.default_rng(6)
    x = rng.normal(size=(2, 6, 7)) * 5 + 3
    y, mean, rstd = O.group_norm(x, 3, None, None, 0.0, return_stats=True)
    grp = y.reshape(2, 3, -1)
    np.testing.assert_allclose(grp.mean(-1), 0, atol=1e-12)
    np.testing.assert_allclose(grp.var(-1), 1, atol=1e-12)
    x2 = x.reshape(2, 3, -1) * np.array([1.5, 0.25, 4.0])[None, :, None] + 11.0
    np.testing.assert_allclose(O.group_norm(x2.reshape(x.shape), 3, None, None, 0.0), y, atol=1e-10)
    silu = O.group_norm(x, 3, None, None, 1e-5, silu=True)
    plain = O.group_norm(x, 3, None, None, 1e-5)
    np.testing.assert_allclose(silu, plain / (1 + np.exp(-plain)), atol=1e-14)


def test_max_rel_err_metric():
    """max|y - ref| / max|ref| (tools/bench_fast.py:147-162 of the reference)."""
    assert O.max_rel_err(np.array([1.0, 2.0, 4.5]), np.array([1.0, 2.0, 4.0])) == pytest.approx(0.125)
    assert O.max_rel_err(np.zeros(3), np.zeros(3)) == 0.0


# ---------------------------------------------------------------------------
# depthwise conv1d backward
# ---------------------------------------------------------------------------
def _stock_dw_grads(x, w, b, pad, l_out, dy):
    """Gradients through stock F.conv1d (float64 autograd) of y = conv1d(pad both sides)[..., :l_out]."""
    xt = torch.tensor(x, requires_grad=True)
    wt = torch.tensor(w[:, None, :], requires_grad=True)
    bt = torch.tensor(b, requires_grad=True)
    K = w.shape[-1]
    L = x.shape[-1]
    right = max(0, l_out + K - 1 - L - pad)
    y = F.conv1d(F.pad(xt, (pad, right)), wt, bt, groups=x.shape[1])[..., :l_out]
    gx, gw, gb = torch.autograd.grad(y, (xt, wt, bt), torch.tensor(dy))
    return gx.numpy(), gw.numpy()[:, 0, :], gb.numpy()


@pytest.mark.parametrize("shape", [(2, 3, 17, 3, 1, 17), (2, 3, 17, 4, 3, 20), (2, 3, 17, 4, 3, 17),
                                   (1, 4, 9, 2, 1, 10), (1, 2, 12, 5, 2, 12), (1, 2, 8, 3, 0, 6)])
def test_dwconv1d_bwd_matches_stock_autograd(shape):
    """Symmetric, causal stock-shape, causal truncated, K=2/5 and 'valid' forms."""
    N, C, L, K, pad, l_out = shape
    rng = np.random.default_rng(sum(shape))
    x, w, b = rng.normal(size=(N, C, L)), rng.normal(size=(C, K)), rng.normal(size=C)
    dy = rng.normal(size=(N, C, l_out))
    got = O.dwconv1d_bwd(x, w, dy, pad)
    for a, r in zip(got, _stock_dw_grads(x, w, b, pad, l_out, dy)):
        np.testing.assert_allclose(a, r, rtol=0, atol=1e-11)


def test_dwconv1d_bwd_brute_force_and_planted_mistakes():
    """Brute force on a tiny case (each gradient = the forward's change per unit change of
    one input, by linearity), and mistakes the pins must catch: a shifted padding, a
    reversed kernel, a dropped batch."""
    rng = np.random.default_rng(9)
    N, C, L, K, pad, l_out = 2, 2, 6, 3, 2, 7
    x, w = rng.normal(size=(N, C, L)), rng.normal(size=(C, K))
    dy = rng.normal(size=(N, C, l_out))
    dx, dw, db = O.dwconv1d_bwd(x, w, dy, pad)
    # d<dy, y>/dx[n,c,s] = <dy, y(e_{n,c,s})> with y linear in x (no bias)
    for n, c, s in itertools.product(range(N), range(C), range(L)):
        e = np.zeros_like(x)
        e[n, c, s] = 1.0
        assert abs((dy * O.dwconv1d(e, w, None, pad, l_out)).sum() - dx[n, c, s]) < 1e-12
    for c, j in itertools.product(range(C), range(K)):
        e = np.zeros_like(w)
        e[c, j] = 1.0
        assert abs((dy * O.dwconv1d(x, e, None, pad, l_out)).sum() - dw[c, j]) < 1e-12
    np.testing.assert_allclose(db, dy.sum(axis=(0, 2)), atol=1e-12)
    assert _far(O.dwconv1d_bwd(x, w, dy, pad - 1)[0], dx)
    assert _far(O.dwconv1d_bwd(x, w[:, ::-1].copy(), dy, pad)[0], dx)
    assert _far(O.dwconv1d_bwd(x, w, dy, pad - 1)[1], dw)
    assert _far(O.dwconv1d_bwd(x[:1], w, dy[:1], pad)[1], dw)


# ---------------------------------------------------------------------------
# GroupNorm backward
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape,G,affine", [((2, 6, 5, 3), 3, True), ((1, 8, 7), 2, False),
                                            ((3, 4, 2, 2, 2), 4, True), ((2, 4, 9), 1, True)])
def test_group_norm_bwd_matches_stock_autograd(shape, G, affine):
    rng = np.random.default_rng(len(shape) * 10 + G)
    x = rng.normal(size=shape) * 2 + 3
    C = shape[1]
    gm, bt = (rng.normal(size=C), rng.normal(size=C)) if affine else (None, None)
    dy = rng.normal(size=shape)
    xt = torch.tensor(x, requires_grad=True)
    params = [torch.tensor(v, requires_grad=True) for v in (gm, bt)] if affine else [None, None]
    y = F.group_norm(xt, G, params[0], params[1], 1e-5)
    want = [xt] + ([params[0], params[1]] if affine else [])
    ref = torch.autograd.grad(y, want, torch.tensor(dy))
    dx, dg, db = O.group_norm_bwd(x, G, gm, dy, 1e-5)
    np.testing.assert_allclose(dx, ref[0].numpy(), rtol=0, atol=1e-10)
    if affine:
        np.testing.assert_allclose(dg, ref[1].numpy(), rtol=0, atol=1e-10)
        np.testing.assert_allclose(db, ref[2].numpy(), rtol=0, atol=1e-10)


def test_group_norm_bwd_identities_and_planted_mistakes():
    """dx sums to zero over each group and is orthogonal to x_hat there (the normalisation
    removes mean and scale); the pins catch a wrong group count, a dropped gamma and a
    wrong eps."""
    rng = np.random.default_rng(17)
    N, C, S, G = 2, 6, 10, 3
    x, gm, dy = rng.normal(size=(N, C, S)), rng.normal(size=C), rng.normal(size=(N, C, S))
    # exact at eps = 0 (with eps, sum x_hat^2 = E var / (var + eps) instead of E)
    dx0 = O.group_norm_bwd(x, G, gm, dy, 0.0)[0]
    xg = x.reshape(N, G, -1)
    xh = (xg - xg.mean(-1, keepdims=True)) / np.sqrt(xg.var(-1, keepdims=True))
    np.testing.assert_allclose(dx0.reshape(N, G, -1).sum(-1), 0, atol=1e-10)
    np.testing.assert_allclose((dx0.reshape(N, G, -1) * xh).sum(-1), 0, atol=1e-9)
    dx, dg, db = O.group_norm_bwd(x, G, gm, dy, 1e-5)
    assert _far(O.group_norm_bwd(x, 2, gm, dy, 1e-5)[0], dx)
    assert _far(O.group_norm_bwd(x, G, None, dy, 1e-5)[0], dx)
    assert _far(O.group_norm_bwd(x, G, gm, dy, 1e-1)[0], dx)
    np.testing.assert_allclose(db, dy.sum(axis=(0, 2)), atol=1e-12)


# ---------------------------------------------------------------------------
# causal conv1d decode step
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("W,silu", [(2, False), (3, True), (4, False), (4, True)])
def test_causal_update_streaming_equals_causal_forward(W, silu):
    """L decode steps from a zero state produce the causal conv of the whole sequence
    (the forward with pad_left = W-1, truncated to L), and leave the last W inputs as the
    state."""
    rng = np.random.default_rng(W * 2 + silu)
    B, D, L = 2, 3, 9
    x, w, b = rng.normal(size=(B, D, L)), rng.normal(size=(D, W)), rng.normal(size=D)
    st = np.zeros((B, D, W))
    ys = []
    for t in range(L):
        y, st = O.causal_conv1d_update(x[:, :, t], st, w, b, silu)
        ys.append(y)
    np.testing.assert_allclose(np.stack(ys, -1), O.dwconv1d(x, w, b, W - 1, L, silu=silu), atol=1e-12)
    np.testing.assert_allclose(st, x[:, :, L - W:], atol=0)


def test_causal_update_planted_mistakes():
    rng = np.random.default_rng(5)
    x, st, w, b = rng.normal(size=(2, 3)), rng.normal(size=(2, 3, 4)), rng.normal(size=(3, 4)), rng.normal(size=3)
    y, s2 = O.causal_conv1d_update(x, st, w, b)
    assert _far(O.causal_conv1d_update(x, st, w[:, ::-1].copy(), b)[0], y)     # reversed taps
    assert _far(O.causal_conv1d_update(x, st, w, None)[0], y)                   # dropped bias
    np.testing.assert_allclose(s2[..., :3], st[..., 1:], atol=0)                 # shift direction
    np.testing.assert_allclose(s2[..., 3], x, atol=0)


# ---------------------------------------------------------------------------
# causal conv with seq_idx / initial / final states (channel-last features)
# ---------------------------------------------------------------------------
def _causal_ref64(x, w, b, init=None, silu=False):
    """The reference's causal_conv1d_ref (causal_conv1d_interface.py:133-172) in float64 on the
    CPU, through the package's stock-PyTorch statement of it."""
    from amd_tuned_torch.causal_conv1d import causal_conv1d_ref
    out = causal_conv1d_ref(x, w, b, initial_states=init, return_final_states=True,
                            activation="silu" if silu else None)
    return out


def _segments(rng, B, L):
    """seq_idx built as the reference's test does (test_causal_conv1d.py:235-245)."""
    lens = []
    for _ in range(B):
        ns = int(rng.integers(1, 5))
        eos = np.sort(rng.permutation(max(L - 1, 1))[:ns]) if L > 1 else np.zeros(0, dtype=int)
        cuts = np.diff(np.concatenate([[-1], eos, [L - 1]]))
        lens.append([int(c) for c in cuts if c > 0])
    seq = np.stack([np.concatenate([np.full(s, i, dtype=np.int32) for i, s in enumerate(sl)]) for sl in lens])
    return lens, seq


@pytest.mark.parametrize("K", [2, 3, 4])
@pytest.mark.parametrize("silu", [False, True])
def test_causal_states_without_states_is_the_causal_conv(K, silu):
    rng = np.random.default_rng(K)
    x, w, b = rng.normal(size=(2, 3, 11)), rng.normal(size=(3, K)), rng.normal(size=3)
    y, fin = O.causal_conv1d_states(x, w, b, silu=silu)
    np.testing.assert_array_equal(y, O.dwconv1d(x, w, b, K - 1, 11, silu))
    np.testing.assert_array_equal(fin, x[..., 11 - (K - 1):])


@pytest.mark.parametrize("K", [2, 3, 4])
@pytest.mark.parametrize("L", [1, 2, 5, 37])
@pytest.mark.parametrize("silu", [False, True])
def test_causal_states_initial_and_final_match_reference_statement(K, L, silu):
    g = torch.Generator().manual_seed(100 * K + L)
    x = torch.randn(2, 4, L, generator=g, dtype=torch.float64)
    w = torch.randn(4, K, generator=g, dtype=torch.float64)
    b = torch.randn(4, generator=g, dtype=torch.float64)
    init = torch.randn(2, 4, K - 1, generator=g, dtype=torch.float64)
    y, fin = O.causal_conv1d_states(x, w, b, initial_states=init, silu=silu)
    ry, rfin = _causal_ref64(x, w, b, init, silu)
    np.testing.assert_allclose(y, ry.numpy(), rtol=0, atol=1e-12)
    np.testing.assert_allclose(fin, rfin.numpy(), rtol=0, atol=0)
    # planted: dropping the initial states must miss the statement
    assert _far(O.causal_conv1d_states(x, w, b, silu=silu)[0], ry.numpy())


@pytest.mark.parametrize("K", [2, 3, 4])
def test_causal_states_seq_idx_matches_per_segment_convs(K):
    """seq_idx == the causal conv of each segment on its own, concatenated (the reference
    test's construction, test_causal_conv1d.py:246-255); an off-by-one seq lookup and a
    reversed kernel are caught."""
    rng = np.random.default_rng(40 + K)
    B, D, L = 3, 4, 29
    lens, seq = _segments(rng, B, L)
    x, w, b = rng.normal(size=(B, D, L)), rng.normal(size=(D, K)), rng.normal(size=D)
    for silu in (False, True):
        y = O.causal_conv1d_states(x, w, b, seq_idx=seq, silu=silu)[0]
        ref = np.concatenate([
            np.concatenate([O.dwconv1d(xs, w, b, K - 1, xs.shape[-1], silu)
                            for xs in np.split(x[[n]], np.cumsum(lens[n])[:-1], axis=2)], axis=2)
            for n in range(B)], axis=0)
        np.testing.assert_allclose(y, ref, rtol=0, atol=1e-12)
        shifted = np.concatenate([seq[:, 1:], seq[:, -1:]], axis=1)
        assert _far(O.causal_conv1d_states(x, w, b, seq_idx=shifted, silu=silu)[0], ref)
        assert _far(O.causal_conv1d_states(x, w[:, ::-1].copy(), b, seq_idx=seq, silu=silu)[0], ref)


@pytest.mark.parametrize("K", [2, 3, 4])
def test_causal_states_streaming(K):
    """Running a sequence in two pieces, the first piece's final states as the second's
    initial states, equals running it whole."""
    rng = np.random.default_rng(70 + K)
    x, w, b = rng.normal(size=(2, 3, 40)), rng.normal(size=(3, K)), rng.normal(size=3)
    init = rng.normal(size=(2, 3, K - 1))
    for cut in (1, K - 1, 17):
        y1, f1 = O.causal_conv1d_states(x[..., :cut], w, b, initial_states=init, silu=True)
        y2, f2 = O.causal_conv1d_states(x[..., cut:], w, b, initial_states=f1, silu=True)
        y, f = O.causal_conv1d_states(x, w, b, initial_states=init, silu=True)
        np.testing.assert_allclose(np.concatenate([y1, y2], axis=-1), y, rtol=0, atol=1e-12)
        np.testing.assert_array_equal(f2, f)


@pytest.mark.parametrize("K", [2, 3, 4])
@pytest.mark.parametrize("L", [1, 2, 9, 33])
@pytest.mark.parametrize("silu", [False, True])
def test_causal_states_bwd_matches_autograd(K, L, silu):
    """dx / dw / db / dinitial_states for upstream gradients on both the output and the
    final states, against float64 autograd of the reference's statement."""
    g = torch.Generator().manual_seed(7 * K + L)
    mk = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)
    x, w, b, init = mk(2, 3, L), mk(3, K), mk(3), mk(2, 3, K - 1)
    dout, dfin = mk(2, 3, L), mk(2, 3, K - 1)
    xr, wr, br, ir = (t.clone().requires_grad_() for t in (x, w, b, init))
    y, fin = _causal_ref64(xr, wr, br, ir, silu)
    ((y * dout).sum() + (fin * dfin).sum()).backward()
    dx, dw, db, dinit = O.causal_conv1d_states_bwd(x, w, b, dout, initial_states=init, dfinal=dfin, silu=silu)
    for a, r in ((dx, xr.grad), (dw, wr.grad), (db, br.grad), (dinit, ir.grad)):
        np.testing.assert_allclose(a, r.numpy(), rtol=0, atol=1e-10)
    # planted: a dropped final-state gradient
    assert _far(O.causal_conv1d_states_bwd(x, w, b, dout, initial_states=init, silu=silu)[3], ir.grad.numpy()) \
        or _far(O.causal_conv1d_states_bwd(x, w, b, dout, initial_states=init, silu=silu)[0], xr.grad.numpy())


@pytest.mark.parametrize("K", [2, 4])
def test_causal_states_bwd_seq_idx_matches_per_segment_autograd(K):
    rng = np.random.default_rng(90 + K)
    B, D, L = 2, 3, 23
    lens, seq = _segments(rng, B, L)
    x, w, b, dout = (torch.from_numpy(rng.normal(size=s)) for s in ((B, D, L), (D, K), (D,), (B, D, L)))
    for silu in (False, True):
        xr, wr, br = (t.clone().requires_grad_() for t in (x, w, b))
        from amd_tuned_torch.causal_conv1d import causal_conv1d_ref
        out = torch.cat([torch.cat([causal_conv1d_ref(xs, wr, br, activation="silu" if silu else None)
                                    for xs in torch.split(xr[[n]], lens[n], dim=2)], dim=2) for n in range(B)])
        (out * dout).sum().backward()
        dx, dw, db, _ = O.causal_conv1d_states_bwd(x, w, b, dout, seq_idx=seq, silu=silu)
        for a, r in ((dx, xr.grad), (dw, wr.grad), (db, br.grad)):
            np.testing.assert_allclose(a, r.numpy(), rtol=0, atol=1e-10)
        assert _far(O.causal_conv1d_states_bwd(x, w, b, dout, silu=silu)[0], xr.grad.numpy())
