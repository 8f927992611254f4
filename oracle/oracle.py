"""Float64 CPU oracle for the hot-path operators -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module, and only as the checker: the product (amd_tuned_torch) never calls it.

Wraps oracle/_build/libatk_oracle.so (plain C, oracle/atk_oracle.c); build with
`make -C oracle` (done by __graft_entry__.build() and, if missing, by `lib()` below).
Every function takes torch tensors or numpy arrays of any float dtype, widens them to
float64 (exact for fp16/bf16/fp32) and returns a float64 numpy array.

Parity pins (tests/test_oracle.py): stock torch.nn.functional in float64 on the CPU (the
reference's own parity target, amd_tuned_torch/kernel_select.py:68-82), brute-force
Python loops on tiny shapes, the committed golden fixtures in tests/golden/, the
depthwise output-length known answers of tests/test_depthwise_conv1d_ops.py:64-71, and
mathematical invariants (delta kernels shift the input, linearity, GroupNorm output has
zero mean / unit variance per group and is invariant to a per-group shift and scale).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "libatk_oracle.so")

_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = ctypes.CDLL(LIB)
        d, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.oracle_dwconv1d.argtypes = [d, d, d, d, i64, i64, i64, i64, i64, i64, i32]
        L.oracle_dwconv1d_bwd.argtypes = [d, d, d, d, d, d, i64, i64, i64, i64, i64, i64]
        L.oracle_causal_conv1d_update.argtypes = [d, d, d, d, d, i64, i64, i64, i32]
        L.oracle_causal_conv1d_states.argtypes = [d, d, d, d, d, d, d, i64, i64, i64, i64, i32]
        L.oracle_causal_conv1d_states_bwd.argtypes = [d] * 11 + [i64, i64, i64, i64, i32]
        L.oracle_group_norm.argtypes = [d, d, d, d, i64, i64, i64, i64, ctypes.c_double, i32, d, d]
        L.oracle_group_norm_bwd.argtypes = [d, d, d, d, d, d, i64, i64, i64, i64, ctypes.c_double]
        L.oracle_conv3d.argtypes = [d, d, d, d] + [i64] * 18 + [d, i64]
        _lib = L
    return _lib


def f64(a) -> np.ndarray:
    """Contiguous float64 numpy copy of a tensor/array (exact widening)."""
    if a is None:
        return None
    try:
        import torch
        if isinstance(a, torch.Tensor):
            a = a.detach().to("cpu", torch.float64).numpy()
    except ImportError:
        pass
    return np.ascontiguousarray(np.asarray(a, dtype=np.float64))


def _p(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def dwconv1d(x, w, b, pad_left: int, l_out: int, silu: bool = False) -> np.ndarray:
    """x [N,C,L], w [C,K] or [C,1,K], b [C] or None."""
    x, w, b = f64(x), f64(w), f64(b)
    N, C, L = x.shape
    w = w.reshape(C, -1)
    y = np.empty((N, C, l_out), dtype=np.float64)
    lib().oracle_dwconv1d(_p(x), _p(w), _p(b), _p(y), N, C, L, w.shape[1], pad_left, l_out,
                          int(bool(silu)))
    return y


def dwconv1d_bwd(x, w, dy, pad_left: int):
    """(dx [N,C,L], dw [C,K], db [C]) of dwconv1d(x, w, b, pad_left, L_out) for the upstream
    gradient dy [N,C,L_out]; w [C,K] or [C,1,K]."""
    x, w, dy = f64(x), f64(w), f64(dy)
    N, C, L = x.shape
    w = w.reshape(C, -1)
    K = w.shape[1]
    dx = np.empty_like(x)
    dw = np.empty((C, K), dtype=np.float64)
    db = np.empty((C,), dtype=np.float64)
    lib().oracle_dwconv1d_bwd(_p(x), _p(w), _p(dy), _p(dx), _p(dw), _p(db), N, C, L, K, pad_left,
                              dy.shape[-1])
    return dx, dw, db


def causal_conv1d_update(x, state, w, b=None, silu: bool = False):
    """(y [B, D], new state [B, D, W]) of one decode step; inputs are not modified."""
    x, w, b = f64(x), f64(w), f64(b)
    st = f64(state).copy()
    B, D = x.shape
    W = w.shape[-1]
    y = np.empty((B, D), dtype=np.float64)
    lib().oracle_causal_conv1d_update(_p(x), _p(st), _p(w.reshape(D, W)), _p(b), _p(y), B, D, W, int(bool(silu)))
    return y, st


def _seq32(seq_idx):
    if seq_idx is None:
        return None
    try:
        import torch
        if isinstance(seq_idx, torch.Tensor):
            seq_idx = seq_idx.detach().cpu().numpy()
    except ImportError:
        pass
    return np.ascontiguousarray(np.asarray(seq_idx, dtype=np.int32))


def causal_conv1d_states(x, w, b=None, seq_idx=None, initial_states=None, silu: bool = False):
    """(y [B, D, L], final_states [B, D, K-1]) of the causal conv with seq_idx [B, L] and
    initial_states [B, D, K-1] (either may be None); layouts are logical, any strides."""
    x, w, b, init = f64(x), f64(w), f64(b), f64(initial_states)
    seq = _seq32(seq_idx)
    B, D, L = x.shape
    K = w.reshape(D, -1).shape[1]
    y = np.empty((B, D, L), dtype=np.float64)
    fin = np.empty((B, D, K - 1), dtype=np.float64)
    lib().oracle_causal_conv1d_states(_p(x), _p(w.reshape(D, K)), _p(b), _p(seq), _p(init), _p(y), _p(fin),
                                      B, D, L, K, int(bool(silu)))
    return y, fin


def causal_conv1d_states_bwd(x, w, b, dout, seq_idx=None, initial_states=None, dfinal=None,
                             silu: bool = False):
    """(dx [B, D, L], dw [D, K], db [D], dinit [B, D, K-1] or None) of causal_conv1d_states
    for the upstream gradients dout and dfinal (None = zero)."""
    x, w, b, dout = f64(x), f64(w), f64(b), f64(dout)
    init, dfin = f64(initial_states), f64(dfinal)
    seq = _seq32(seq_idx)
    B, D, L = x.shape
    K = w.reshape(D, -1).shape[1]
    dx = np.empty_like(x)
    dw = np.empty((D, K), dtype=np.float64)
    db = np.empty((D,), dtype=np.float64)
    dinit = np.empty((B, D, K - 1), dtype=np.float64) if init is not None else None
    lib().oracle_causal_conv1d_states_bwd(_p(x), _p(w.reshape(D, K)), _p(b), _p(seq), _p(init), _p(dout),
                                          _p(dfin), _p(dx), _p(dw), _p(db), _p(dinit), B, D, L, K,
                                          int(bool(silu)))
    return dx, dw, db, dinit


def conv1d_out_len(length: int, padding: int, width: int) -> int:
    return length + 2 * padding - width + 1


def group_norm(x, G: int, gamma=None, beta=None, eps: float = 1e-5, silu: bool = False,
               return_stats: bool = False):
    x, gamma, beta = f64(x), f64(gamma), f64(beta)
    N, C = x.shape[0], x.shape[1]
    S = int(np.prod(x.shape[2:])) if x.ndim > 2 else 1
    y = np.empty_like(x)
    mean = np.empty(N * G)
    rstd = np.empty(N * G)
    lib().oracle_group_norm(_p(x), _p(gamma), _p(beta), _p(y), N, C, S, G, float(eps),
                            int(bool(silu)), _p(mean), _p(rstd))
    if return_stats:
        return y, mean.reshape(N, G), rstd.reshape(N, G)
    return y


def group_norm_bwd(x, G: int, gamma, dy, eps: float = 1e-5):
    """(dx, dgamma [C], dbeta [C]) of group_norm(x, G, gamma, beta, eps) for dy (x's shape)."""
    x, gamma, dy = f64(x), f64(gamma), f64(dy)
    N, C = x.shape[:2]
    S = x.size // (N * C) if N * C else 0
    dx = np.empty_like(x)
    dg = np.empty((C,), dtype=np.float64)
    db = np.empty((C,), dtype=np.float64)
    lib().oracle_group_norm_bwd(_p(x), _p(gamma), _p(dy), _p(dx), _p(dg), _p(db), N, C, S, G, eps)
    return dx, dg, db


def _t3(v):
    return (v, v, v) if isinstance(v, int) else tuple(v)


def conv_out_shape(xshape, wshape, stride, padding, dilation):
    nd = len(xshape) - 2
    s = (stride,) * nd if isinstance(stride, int) else tuple(stride)
    p = (padding,) * nd if isinstance(padding, int) else tuple(padding)
    d = (dilation,) * nd if isinstance(dilation, int) else tuple(dilation)
    sp = [(i + 2 * pp - dd * (k - 1) - 1) // ss + 1
          for i, k, ss, pp, dd in zip(xshape[2:], wshape[2:], s, p, d)]
    return (xshape[0], wshape[0], *sp)


def conv3d(x, w, b=None, stride=1, padding=0, dilation=1, points=None) -> np.ndarray:
    """Dense NCDHW conv3d (groups = 1).  `points`: optional flat output indices to compute
    (returns a 1-D array for them); otherwise the full output."""
    x, w, b = f64(x), f64(w), f64(b)
    N, Ci, D, H, W = x.shape
    Co, _, KD, KH, KW = w.shape
    s, p, d = _t3(stride), _t3(padding), _t3(dilation)
    oshape = conv_out_shape(x.shape, w.shape, s, p, d)
    if points is None:
        n = int(np.prod(oshape))
        y = np.empty(n)
        pts = None
    else:
        pts = np.ascontiguousarray(np.asarray(points, dtype=np.int64))
        n = pts.size
        y = np.empty(n)
    lib().oracle_conv3d(_p(x), _p(w), _p(b), _p(y), N, Ci, D, H, W, Co, KD, KH, KW, *s, *p, *d,
                        None if pts is None else pts.ctypes.data_as(ctypes.c_void_p), n)
    return y if points is not None else y.reshape(oshape)


def conv2d(x, w, b=None, stride=1, padding=0, dilation=1, points=None) -> np.ndarray:
    """Dense NCHW conv2d as the D = KD = 1 case of conv3d."""
    x, w = f64(x), f64(w)
    s = (stride, stride) if isinstance(stride, int) else tuple(stride)
    p = (padding, padding) if isinstance(padding, int) else tuple(padding)
    d = (dilation, dilation) if isinstance(dilation, int) else tuple(dilation)
    y = conv3d(x[:, :, None], w[:, :, None], b, (1, *s), (0, *p), (1, *d), points=points)
    return y if points is not None else y[:, :, 0]


def max_rel_err(y, y_ref) -> float:
    """max|y - y_ref| / max|y_ref| -- the metric of the reference's benchmark
    (tools/bench_fast.py:147-162) and of the parity bars."""
    y, y_ref = f64(y), f64(y_ref)
    denom = float(np.max(np.abs(y_ref))) if y_ref.size else 0.0
    num = float(np.max(np.abs(y - y_ref))) if y.size else 0.0
    return num / denom if denom > 0 else num
