"""CPU checks of causal_conv1d_fn / CausalConv1dFn's argument handling against the
reference interface (src/causal-conv1d-amd/causal_conv1d/causal_conv1d_interface.py:10-130,
host checks causal_conv1d.cpp:155-222): every case here is rejected before any device work,
so no GPU is needed."""
from __future__ import annotations

import pytest
import torch

from amd_tuned_torch import causal_conv1d as cc


def _cl(batch=2, dim=16, seqlen=8):
    """x (batch, dim, seqlen) with x.stride(1) == 1: the reference's channel-last layout."""
    return torch.randn(batch, seqlen, dim).transpose(1, 2)


def test_channel_last_predicate_matches_reference():
    assert cc._channel_last(_cl())
    assert not cc._channel_last(torch.randn(2, 16, 8))
    # a freshly allocated length-1 sequence has stride(2) == 1: the (B, C, L) kernel, as in the
    # reference; a transposed view keeps its stride(2) and counts as channel-last in both
    assert not cc._channel_last(torch.randn(2, 16, 1))
    assert cc._channel_last(torch.randn(2, 1, 16).transpose(1, 2))


def test_activation_must_be_silu_swish_or_none():
    with pytest.raises(NotImplementedError):
        cc.causal_conv1d_fn(torch.randn(2, 16, 8), torch.randn(16, 4), activation="relu")


def test_width_limits():
    with pytest.raises(RuntimeError, match="width between 2 and 4"):
        cc.causal_conv1d_fn(torch.randn(2, 16, 8), torch.randn(16, 5))
    with pytest.raises(RuntimeError, match="width between 2 and 4"):
        cc.causal_conv1d_fn(torch.randn(2, 16, 8), torch.randn(16, 1))


def test_seq_idx_excludes_states():
    seq = torch.zeros(2, 8, dtype=torch.int32)
    with pytest.raises(AssertionError, match="initial_states must be None"):
        cc.causal_conv1d_fn(_cl(), torch.randn(16, 4), seq_idx=seq, initial_states=torch.randn(2, 16, 3))
    with pytest.raises(AssertionError, match="don't return final_states"):
        cc.causal_conv1d_fn(_cl(), torch.randn(16, 4), seq_idx=seq, return_final_states=True)


def test_final_states_need_channel_last():
    with pytest.raises(AssertionError, match="channel-last"):
        cc.causal_conv1d_fn(torch.randn(2, 16, 8), torch.randn(16, 4), return_final_states=True)


@pytest.mark.parametrize("kw,msg", [
    ({"seq_idx": torch.zeros(2, 8, dtype=torch.int32)}, "seq_idx is only supported for channel last layout"),
    ({"initial_states": torch.randn(2, 16, 3)}, "initial_states is only supported for channel last layout"),
])
def test_bcl_layout_rejects_channel_last_features(kw, msg):
    """On a (B, C, L) x the reference's host code rejects seq_idx / initial_states
    (causal_conv1d.cpp:173,195); so does this package, with the same messages."""
    with pytest.raises(RuntimeError, match=msg):
        cc.causal_conv1d_fn(torch.randn(2, 16, 8), torch.randn(16, 4), **kw)


def test_ref_statements_agree_with_each_other():
    """causal_conv1d_ref with initial states equals the plain ref on the concatenated sequence
    (its own definition), and the decode ref reproduces the last column of the full ref."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 16, 10, generator=g, dtype=torch.float64)
    w = torch.randn(16, 4, generator=g, dtype=torch.float64)
    b = torch.randn(16, generator=g, dtype=torch.float64)
    init = torch.randn(2, 16, 3, generator=g, dtype=torch.float64)
    y, fin = cc.causal_conv1d_ref(x, w, b, initial_states=init, return_final_states=True, activation="silu")
    y_all = cc.causal_conv1d_ref(torch.cat([init, x], dim=-1), w, b, activation="silu")[..., 3:]
    torch.testing.assert_close(y, y_all)
    torch.testing.assert_close(fin, x[..., -3:])
    state = torch.cat([torch.zeros(2, 16, 1, dtype=torch.float64), x[..., -4:-1]], dim=-1)
    step = cc.causal_conv1d_update_ref(x[..., -1], state, w, b, activation="silu")
    torch.testing.assert_close(step, cc.causal_conv1d_ref(x, w, b, activation="silu")[..., -1])
