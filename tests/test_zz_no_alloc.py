"""The no-allocation GroupNorm entry point (atk_group_norm_fwd_noalloc, static per-GPU
scratch) against the workspace entry point (atk_group_norm_fwd) through the C ABI: the same
kernels and arithmetic, so the outputs must be identical byte for byte -- over two calls in
a row, the second on a smaller input, for a multi-slice register-resident variant (slot
table in the scratch) and the two-pass variant (partials in the scratch); calls on two streams
that may overlap (each stream has its own slice of the scratch); and the refusal of a stream
beyond the slices."""
from __future__ import annotations

import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _native():
    from amd_tuned_torch import _native
    return _native


def _inputs(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    C = shape[1]
    mu = (torch.rand(C, generator=g) * 4 - 2).reshape(1, C, *([1] * (len(shape) - 2)))
    x = (torch.randn(shape, generator=g) + mu).to(dtype)
    gm = (1 + 0.1 * torch.randn(C, generator=g)).to(dtype)
    bt = (0.1 * torch.randn(C, generator=g)).to(dtype)
    return x, gm, bt


@pytest.mark.parametrize("name", ["res_nt256_v8", "res_nt512_v16", "twopass"])
def test_group_norm_noalloc_matches_workspace_entry_point(dev, name):
    nat = _native()
    vi = nat.variants(nat.OP_GROUP_NORM).index(name)
    # first a large call (many slices per group: the slot table / partials are used), then a
    # smaller one that must not see anything the first left in the scratch
    for shape, G, silu, seed in (((1, 64, 32, 32, 64), 32, True, 3), ((2, 32, 16, 16), 8, False, 4)):
        x, gm, bt = _inputs(shape, torch.bfloat16, seed)
        xd, gd, bd = x.to(dev), gm.to(dev), bt.to(dev)
        want = nat.group_norm(xd, G, gd, bd, 1e-5, silu=silu, variant=vi)
        out = torch.empty_like(xd)
        torch.cuda.synchronize()
        before = torch.cuda.memory_stats(dev).get("allocation.all.allocated", 0)
        got = nat.group_norm_noalloc(xd, G, out, gd, bd, 1e-5, silu=silu, variant=vi)
        torch.cuda.synchronize()
        assert torch.cuda.memory_stats(dev).get("allocation.all.allocated", 0) == before
        assert got is out
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (name, shape)
        assert O.max_rel_err(got.cpu(), O.group_norm(x, G, gm, bt, 1e-5, silu=silu)) <= 1e-2
    assert not nat.group_norm_barrier_error(dev)


def test_group_norm_noalloc_rejects_shapes_beyond_the_scratch(dev):
    """Two-pass partials above the static scratch's 1 MiB (262144 groups here) are refused
    with a clear error; nothing is launched."""
    nat = _native()
    vi = nat.variants(nat.OP_GROUP_NORM).index("twopass")
    x = torch.zeros(8192, 32, 16, dtype=torch.float16, device=dev)
    out = torch.empty_like(x)
    with pytest.raises(RuntimeError, match="static scratch holds"):
        nat.group_norm_noalloc(x, 32, out, None, None, 1e-5, variant=vi)
    assert nat.lib().atk_group_norm_noalloc_scratch_bytes() > (1 << 20)


def test_group_norm_noalloc_overlapping_streams_use_their_own_slices(dev):
    """Calls on two streams, issued back to back so that they may overlap on the GPU, each use
    the scratch slice bound to their stream: both results equal the workspace entry point's
    bit for bit, over several rounds (multi-slice resident variant: slot table in the scratch;
    two-pass: partials)."""
    nat = _native()
    s1, s2 = torch.cuda.Stream(dev), torch.cuda.Stream(dev)
    for name in ("res_nt256_v8", "twopass"):
        vi = nat.variants(nat.OP_GROUP_NORM).index(name)
        ins = [_inputs((1, 64, 32, 32, 64), torch.bfloat16, 11), _inputs((1, 64, 32, 32, 64), torch.bfloat16, 12)]
        dins = [tuple(t.to(dev) for t in xi) for xi in ins]
        wants = [nat.group_norm(xd, 32, gd, bd, 1e-5, silu=True, variant=vi) for xd, gd, bd in dins]
        outs = [torch.empty_like(xd) for xd, _, _ in dins]
        torch.cuda.synchronize()
        for _ in range(3):
            for st, (xd, gd, bd), out in zip((s1, s2), dins, outs):
                with torch.cuda.stream(st):
                    nat.group_norm_noalloc(xd, 32, out, gd, bd, 1e-5, silu=True, variant=vi)
            torch.cuda.synchronize()
            for out, want in zip(outs, wants):
                assert torch.equal(out.view(torch.int16), want.view(torch.int16)), name
    for (x, gm, bt), out in zip(ins, outs):
        assert O.max_rel_err(out.cpu(), O.group_norm(x, 32, gm, bt, 1e-5, silu=True)) <= 1e-2
    assert not nat.group_norm_barrier_error(dev)


def test_group_norm_noalloc_refuses_a_stream_beyond_its_slices(dev):
    """Once every slice of the GPU's scratch is bound to a stream, a call from a further
    stream is refused with a clear error (it would race on a bound slice); streams that hold
    a slice keep working.  Runs last: it leaves every slice bound for the process."""
    nat = _native()
    vi = nat.variants(nat.OP_GROUP_NORM).index("res_nt256_v8")
    x, gm, bt = (t.to(dev) for t in _inputs((2, 32, 16, 16), torch.bfloat16, 5))
    want = nat.group_norm(x, 8, gm, bt, 1e-5, variant=vi)
    torch.cuda.synchronize()  # the inputs and the reference are ready before other streams read them
    streams, refused = [], None
    for i in range(5):
        st = torch.cuda.Stream(dev)
        streams.append(st)
        out = torch.empty_like(x)
        with torch.cuda.stream(st):
            try:
                nat.group_norm_noalloc(x, 8, out, gm, bt, 1e-5, variant=vi)
            except RuntimeError as exc:
                assert "stream slices" in str(exc)
                refused = i
                break
        st.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    assert refused is not None, "a fifth stream was given a slice of a 4-slice scratch"
    if refused > 0:
        out = torch.empty_like(x)
        with torch.cuda.stream(streams[0]):
            nat.group_norm_noalloc(x, 8, out, gm, bt, 1e-5, variant=vi)
        streams[0].synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16))
