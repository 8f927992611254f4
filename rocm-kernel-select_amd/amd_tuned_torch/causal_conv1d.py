"""Causal depthwise conv1d (Mamba-style), forward and backward.

Interface of the `causal_conv1d` package the reference imports for its conv1d fast path
(src/causal-conv1d-amd/causal_conv1d/causal_conv1d_interface.py:10-130):

    causal_conv1d_fn(x, weight, bias=None, seq_idx=None, initial_states=None,
                     return_final_states=False, final_states_out=None, activation=None)
    x: (batch, dim, seqlen), weight: (dim, width), bias: (dim,) -> out: (batch, dim, seqlen)

out[b,c,t] = act(bias[c] + sum_j weight[c,j] * x[b,c,t-(width-1)+j]), x < 0 taken as zero
(or from initial_states); act is SiLU for activation "silu"/"swish".  As in the reference
(causal_conv1d.cpp:155-222) the layout decides the kernel: x.stride(1) == 1 with
x.stride(2) > 1 is channel-last and runs the channels-last kernel, which also serves seq_idx
(taps across a sequence boundary dropped) and initial / final states; any other x runs the
(B, C, L) kernel and rejects those three.  Weights given in fp32 are used unrounded by both
layouts and by the decode step, as the reference dispatches the weight type separately
(causal_conv1d.cpp:139-141,229,437); weights of another type are used in x's dtype.  The backward (the
reference's causal_conv1d_bwd) is one fused channels-last kernel (dx, dweight, dbias, with the
SiLU derivative from the recomputed fp32 pre-activation); the (B, C, L) layout composes the
forward kernel on the flipped weights with the weight-gradient kernel.  The decode step
`causal_conv1d_update(x, conv_state, weight, bias, activation)` (interface :175-213) runs the
library's update kernel.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _native


def _channel_last(x: torch.Tensor) -> bool:
    """The reference's layout test (causal_conv1d.cpp:156)."""
    return x.stride(1) == 1 and x.stride(2) > 1


def _kernel_weight(weight: torch.Tensor, x: torch.Tensor, bias):
    """The weights (and bias) as the kernels take them: fp32, or x's dtype."""
    w = weight if weight.dtype in (torch.float32, x.dtype) else weight.float()
    return w, (bias.to(w.dtype) if bias is not None else None)


def _forward(x, weight, bias, seq_idx, initial_states, final_states_out, silu: bool):
    B, D, L = x.shape
    K = weight.shape[1]
    if _channel_last(x):
        w, b = _kernel_weight(weight, x, bias)
        out = torch.empty_like(x)
        _native.dwconv1d_cl(
            x.transpose(1, 2), w, b, K - 1, L, silu=silu, seq_idx=seq_idx,
            seq_mode=1 if seq_idx is not None else 0,
            initial_states=None if initial_states is None else initial_states.transpose(1, 2),
            final_states=None if final_states_out is None else final_states_out.transpose(1, 2),
            out=out.transpose(1, 2))
        return out
    if seq_idx is not None:
        raise RuntimeError("seq_idx is only supported for channel last layout")
    if initial_states is not None:
        raise RuntimeError("initial_states is only supported for channel last layout")
    if final_states_out is not None:
        raise RuntimeError("final_states is only supported for channel last layout")
    w, b = _kernel_weight(weight, x, bias)
    return _native.dwconv1d(x.contiguous(), w.contiguous(), b, K - 1, L, silu=silu)


def _dsilu(z: torch.Tensor) -> torch.Tensor:
    s = torch.sigmoid(z)
    return s * (1 + z * (1 - s))


def _backward(x, weight, bias, dout, seq_idx, initial_states, dfinal, silu: bool, want_dinit: bool):
    """(dx, dweight, dbias, dinitial_states) -- the reference's causal_conv1d_bwd
    (causal_conv1d.cpp:240-380)."""
    B, D, L = x.shape
    K = weight.shape[1]
    if _channel_last(x):
        if dout.stride(1) != 1:
            dout = dout.transpose(-1, -2).contiguous().transpose(-1, -2)
        w, b = _kernel_weight(weight, x, bias)
        dx = torch.empty_like(x)
        _, dw, db = _native.causal_conv1d_cl_bwd(
            x.transpose(1, 2), dout.transpose(1, 2), w, b, silu=silu, seq_idx=seq_idx,
            initial_states=None if initial_states is None else initial_states.transpose(1, 2),
            dx=dx.transpose(1, 2))
    else:
        # differentiate the function the forward computed: weights and bias as the kernel took them
        xc, g = x.contiguous(), dout.contiguous()
        wq, bq = _kernel_weight(weight, x, bias)
        wq = wq.contiguous()
        fused = None
        try:
            fused = _native.causal_conv1d_bwd(xc, g, wq, bq, silu=silu)
        except _native.Unsupported:
            fused = None
        if fused is not None:
            dx, dw, db = fused
        elif silu:
            # the SiLU derivative needs the fp32 pre-activation: run both kernels in fp32
            xf, wf = xc.float(), wq.float()
            z = _native.dwconv1d(xf, wf, bq.float() if bq is not None else None, K - 1, L)
            gf = g.float() * _dsilu(z)
            dx = _native.dwconv1d(gf, wf.flip(-1).contiguous(), None, 0, L).to(x.dtype)
            dw, db = _native.dwconv1d_bwd_weight(xf, gf, K, K - 1)
        else:
            dx = _native.dwconv1d(g, wq.flip(-1).contiguous(), None, 0, L)
            dw, db = _native.dwconv1d_bwd_weight(xc, g, K, K - 1)
    dinit = None
    if initial_states is not None and want_dinit:
        # positions -(K-1)..-1: dinit[q] = sum_{t <= q} w[q - t] * g[t], g the gradient of the
        # pre-activation at the first K-1 outputs (recomputed here on tiny slices)
        n = min(K - 1, L)
        wf = weight.float()
        g = dout[..., :n].float()
        if silu:
            xcat = torch.cat([initial_states.float(), x[..., :n].float()], dim=-1)
            z = sum(wf[:, j, None] * xcat[..., j:j + n] for j in range(K))
            if bias is not None:
                z = z + bias.float()[:, None]
            g = g * _dsilu(z)
        dinit32 = torch.zeros(B, D, K - 1, dtype=torch.float32, device=x.device)
        for q in range(K - 1):
            for t in range(min(q, n - 1) + 1):
                dinit32[..., q] += wf[:, q - t] * g[..., t]
        dinit = torch.empty(B, K - 1, D, dtype=x.dtype, device=x.device).transpose(1, 2)
        dinit.copy_(dinit32)
    if dfinal is not None:
        # final_states[j] = x at position L - (K-1) + j (initial state when negative)
        for j in range(K - 1):
            p = L - (K - 1) + j
            if p >= 0:
                dx[..., p] += dfinal[..., j].to(dx.dtype)
            elif dinit is not None:
                dinit[..., p + K - 1] += dfinal[..., j].to(dinit.dtype)
    return dx, dw.to(weight.dtype), (db.to(bias.dtype) if bias is not None else None), dinit


class CausalConv1dFn(torch.autograd.Function):
    """The reference's CausalConv1dFn (causal_conv1d_interface.py:10-98): same argument
    checks, same saved tensors, same gradient outputs."""

    @staticmethod
    def forward(ctx, x, weight, bias=None, seq_idx=None, initial_states=None, return_final_states=False,
                final_states_out=None, activation=None):
        if activation not in (None, "silu", "swish"):
            raise NotImplementedError("activation must be None, silu, or swish")
        if x.dim() != 3 or weight.dim() != 2 or weight.shape[0] != x.shape[1]:
            raise RuntimeError("causal_conv1d_fn: expects x (batch, dim, seqlen), weight (dim, width)")
        if not 2 <= weight.shape[1] <= 4:
            raise RuntimeError("causal_conv1d only supports width between 2 and 4")
        if x.stride(2) != 1 and x.stride(1) != 1:
            x = x.contiguous()
        bias = bias.contiguous() if bias is not None else None
        if seq_idx is not None:
            assert initial_states is None, "initial_states must be None if seq_idx is not None"
            assert not return_final_states, "If seq_idx is not None, we don't return final_states_out"
        seq_idx = seq_idx.contiguous() if seq_idx is not None else None
        if initial_states is not None and initial_states.stride(2) != 1 and initial_states.stride(1) != 1:
            initial_states = initial_states.contiguous()
        if return_final_states:
            assert x.stride(1) == 1, "Only channel-last layout support returning final_states_out"
            if final_states_out is not None:
                assert final_states_out.stride(2) == 1 or final_states_out.stride(1) == 1
            else:
                batch, dim, _ = x.shape
                width = weight.shape[1]
                final_states_out = torch.empty(batch, width - 1, dim, device=x.device,
                                               dtype=x.dtype).transpose(1, 2)
        else:
            final_states_out = None
        ctx.activation = activation in ("silu", "swish")
        out = _forward(x, weight, bias, seq_idx, initial_states, final_states_out, ctx.activation)
        ctx.save_for_backward(x, weight, bias, seq_idx, initial_states)
        ctx.return_final_states = return_final_states
        ctx.return_dinitial_states = initial_states is not None and initial_states.requires_grad
        return out if not return_final_states else (out, final_states_out)

    @staticmethod
    def backward(ctx, dout, *args):
        x, weight, bias, seq_idx, initial_states = ctx.saved_tensors
        dfinal = args[0] if ctx.return_final_states else None
        if dout.stride(2) != 1 and dout.stride(1) != 1:
            dout = dout.contiguous()
        dx, dweight, dbias, dinit = _backward(x, weight, bias, dout, seq_idx, initial_states, dfinal,
                                              ctx.activation, ctx.return_dinitial_states)
        return (dx, dweight, dbias if bias is not None else None, None,
                dinit if initial_states is not None else None, None, None, None)


def causal_conv1d_fn(x, weight, bias=None, seq_idx=None, initial_states=None,
                     return_final_states=False, final_states_out=None, activation=None):
    """x (batch, dim, seqlen), weight (dim, width), bias (dim,), seq_idx int32 (batch, seqlen),
    initial_states / final_states_out (batch, dim, width - 1); returns out, or (out,
    final_states) with return_final_states (causal_conv1d_interface.py:100-130)."""
    return CausalConv1dFn.apply(x, weight, bias, seq_idx, initial_states, return_final_states,
                                final_states_out, activation)


def _check_activation(activation) -> None:
    if activation not in (None, "silu", "swish"):
        raise NotImplementedError("activation must be None, silu, or swish")


def causal_conv1d_ref(x, weight, bias=None, initial_states=None, return_final_states=False,
                      final_states_out=None, activation=None):
    """Stock-PyTorch statement of causal_conv1d_fn (the reference keeps one beside its kernel,
    causal_conv1d_interface.py:133-172): in the weight's dtype, the sequence is prefixed by
    its width-1 positions of left context -- initial_states, or zeros -- and a 'valid'
    depthwise F.conv1d over that gives the seqlen outputs; final states are the last width-1
    positions of the prefixed sequence."""
    _check_activation(activation)
    dim, width = weight.shape
    context = (initial_states if initial_states is not None
               else x.new_zeros((x.shape[0], dim, width - 1)))
    prefixed = torch.cat([context.to(weight.dtype), x.to(weight.dtype)], dim=-1)
    out = F.conv1d(prefixed, weight.unsqueeze(1), bias, groups=dim)
    if activation is not None:
        out = F.silu(out)
    out = out.to(x.dtype)
    if not return_final_states:
        return out
    tail = prefixed[..., prefixed.shape[-1] - (width - 1):].to(x.dtype)
    if final_states_out is not None:
        tail = final_states_out.copy_(tail)
    return out, tail


def causal_conv1d_update(x, conv_state, weight, bias=None, activation=None):
    """One decode step (causal_conv1d_interface.py:175-189):
    x (batch, dim), conv_state (batch, dim, width) updated in place, weight (dim, width),
    bias (dim,) -> out (batch, dim)."""
    if activation not in (None, "silu", "swish"):
        raise NotImplementedError("activation must be None, silu, or swish")
    width = weight.shape[-1]
    if not 2 <= width <= 4:
        raise RuntimeError("causal_conv1d only supports width between 2 and 4")
    weight, bias = _kernel_weight(weight, x, bias)
    return _native.causal_conv1d_update(x, conv_state, weight, bias, silu=activation is not None)


def causal_conv1d_update_ref(x, conv_state, weight, bias=None, activation=None):
    """Stock-PyTorch statement of the decode step (the reference keeps one beside its kernel,
    causal_conv1d_interface.py:192-213): the state window slides one position, x entering
    at the newest end (conv_state is updated in place), and the output is the window's dot
    product with the weights, plus bias, optionally SiLU, in x's dtype."""
    _check_activation(activation)
    batch, dim = x.shape
    if conv_state.shape != (batch, dim, weight.shape[1]) or weight.shape[0] != dim:
        raise AssertionError("conv_state must be (batch, dim, width) and weight (dim, width)")
    window = torch.cat([conv_state[..., 1:], x.unsqueeze(-1).to(conv_state.dtype)], dim=-1)
    conv_state.copy_(window)
    out = (conv_state * weight).sum(dim=-1)
    if bias is not None:
        out = out + bias
    if activation is not None:
        out = F.silu(out)
    return out.to(x.dtype)
