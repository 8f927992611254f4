"""Causal depthwise conv1d (Mamba-style), forward.

Interface of the `causal_conv1d` package the reference imports for its conv1d fast path
(src/causal-conv1d-amd/causal_conv1d/causal_conv1d_interface.py:100-172):

    causal_conv1d_fn(x, weight, bias=None, seq_idx=None, initial_states=None,
                     return_final_states=False, final_states_out=None, activation=None)
    x: (batch, dim, seqlen), weight: (dim, width), bias: (dim,) -> out: (batch, dim, seqlen)

out[b,c,t] = act(bias[c] + sum_j weight[c,j] * x[b,c,t-(width-1)+j]), x < 0 taken as zero;
act is SiLU for activation "silu"/"swish".  The forward runs the gfx950 depthwise kernel
with pad_left = width - 1 and output length seqlen (the SiLU fused in its epilogue).  The
reference's host limits (causal_conv1d.cpp:157-162: width 2..4) are kept.  seq_idx,
initial_states and final states are channel-last features of the reference kernel and are
not built here (NotImplementedError).  The decode step `causal_conv1d_update(x, conv_state,
weight, bias, activation)` (interface :175-213) runs the library's update kernel.  The
backward of the full-sequence form is the depthwise conv1d backward of the F.conv1d path.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _native


def causal_conv1d_fn(x, weight, bias=None, seq_idx=None, initial_states=None,
                     return_final_states=False, final_states_out=None, activation=None):
    if activation not in (None, "silu", "swish"):
        raise NotImplementedError("activation must be None, silu, or swish")
    if seq_idx is not None or initial_states is not None or return_final_states or \
            final_states_out is not None:
        raise NotImplementedError("seq_idx / initial_states / final_states are not built")
    if x.dim() != 3 or weight.dim() != 2 or weight.shape[0] != x.shape[1]:
        raise RuntimeError("causal_conv1d_fn: expects x (batch, dim, seqlen), weight (dim, width)")
    width = weight.shape[1]
    if not 2 <= width <= 4:
        raise RuntimeError("causal_conv1d only supports width between 2 and 4")
    if weight.dtype != x.dtype:
        weight = weight.to(x.dtype)
    if bias is not None and bias.dtype != x.dtype:
        bias = bias.to(x.dtype)
    x = x.contiguous()
    return _native.dwconv1d(x, weight, bias, width - 1, x.shape[-1], silu=activation is not None)


def causal_conv1d_ref(x, weight, bias=None, initial_states=None, return_final_states=False,
                      final_states_out=None, activation=None):
    """Stock-PyTorch statement of the same operator (the reference's causal_conv1d_ref)."""
    if activation not in (None, "silu", "swish"):
        raise NotImplementedError("activation must be None, silu, or swish")
    dtype_in = x.dtype
    x = x.to(weight.dtype)
    seqlen = x.shape[-1]
    dim, width = weight.shape
    if initial_states is None:
        out = F.conv1d(x, weight.unsqueeze(1), bias, padding=width - 1, groups=dim)
    else:
        x = torch.cat([initial_states, x], dim=-1)
        out = F.conv1d(x, weight.unsqueeze(1), bias, padding=0, groups=dim)
    out = out[..., :seqlen]
    final_states = None
    if return_final_states:
        final_states = F.pad(x, (width - 1 - x.shape[-1], 0)).to(dtype_in)
        if final_states_out is not None:
            final_states_out.copy_(final_states)
            final_states = final_states_out
    out = (out if activation is None else F.silu(out)).to(dtype=dtype_in)
    return out if not return_final_states else (out, final_states)


def causal_conv1d_update(x, conv_state, weight, bias=None, activation=None):
    """One decode step (causal_conv1d_interface.py:175-189):
    x (batch, dim), conv_state (batch, dim, width) updated in place, weight (dim, width),
    bias (dim,) -> out (batch, dim)."""
    if activation not in (None, "silu", "swish"):
        raise NotImplementedError("activation must be None, silu, or swish")
    width = weight.shape[-1]
    if not 2 <= width <= 4:
        raise RuntimeError("causal_conv1d only supports width between 2 and 4")
    if weight.dtype != x.dtype:
        weight = weight.to(x.dtype)
    if bias is not None and bias.dtype != x.dtype:
        bias = bias.to(x.dtype)
    return _native.causal_conv1d_update(x, conv_state, weight, bias, silu=activation is not None)


def causal_conv1d_update_ref(x, conv_state, weight, bias=None, activation=None):
    """Stock-PyTorch statement of the decode step (the reference's causal_conv1d_update_ref,
    causal_conv1d_interface.py:192-213)."""
    if activation not in (None, "silu", "swish"):
        raise NotImplementedError("activation must be None, silu, or swish")
    dtype_in = x.dtype
    batch, dim = x.shape
    width = weight.shape[1]
    assert conv_state.shape == (batch, dim, width)
    assert weight.shape == (dim, width)
    conv_state.copy_(torch.roll(conv_state, shifts=-1, dims=-1))
    conv_state[:, :, -1] = x
    out = torch.sum(conv_state * weight, dim=-1)
    if bias is not None:
        out += bias
    return (out if activation is None else F.silu(out)).to(dtype=dtype_in)
