"""GPU tests of the host path's argument blocks (atk_*_args entry points): the block forms give
the positional entry points' results bit for bit, the per-shape conv plans follow the shape,
dtype and variant (and plan unhashable arguments too), and calls from several Python threads
at once -- ctypes releases the GIL during the call, and each thread fills its own block --
match single-threaded results bit for bit."""
from __future__ import annotations

import ctypes
import threading

import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _nat():
    from amd_tuned_torch import _native
    return _native


def _conv_case(dev, shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g).to(dtype).to(dev)
    w = (torch.randn(shape[1], shape[1], 3, 3, 3, generator=g) * 0.1).to(dtype).to(dev)
    b = (0.1 * torch.randn(shape[1], generator=g)).to(dtype).to(dev)
    return x, w, b


def _mfma_variant(nat, dtype):
    names = nat.variants(nat.OP_CONV)
    return names.index("h_w22_f11_cb32_k2" if dtype != torch.float32 else "f32_w22_f11_cb16_k2")


def test_blocks_match_positional_entry_points(dev):
    """dwconv1d, GroupNorm and the prepacked conv through their argument blocks against the
    same call through the positional entry point on the same buffers: bit-identical."""
    nat = _nat()
    L = nat.lib()
    g = torch.Generator().manual_seed(11)
    # dwconv1d
    x = torch.randn(2, 8, 300, generator=g).to(torch.bfloat16).to(dev)
    w = torch.randn(8, 4, generator=g).to(torch.bfloat16).to(dev)
    b = torch.randn(8, generator=g).to(torch.bfloat16).to(dev)
    y1 = nat.dwconv1d(x, w, b, 3, 303)
    y2 = torch.empty_like(y1)
    rc = L.atk_dwconv1d_fwd(x.data_ptr(), w.data_ptr(), b.data_ptr(), y2.data_ptr(), 2, 8, 300, 4, 3, 303,
                            nat._DTYPE_CODE[x.dtype], nat._DTYPE_CODE[w.dtype], 0, -1, nat._stream(x))
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    # GroupNorm (the workspace the block call used)
    xg = torch.randn(2, 32, 16, 16, generator=g).to(torch.float16).to(dev)
    gm = torch.randn(32, generator=g).to(torch.float16).to(dev)
    bt = torch.randn(32, generator=g).to(torch.float16).to(dev)
    z1 = nat.group_norm(xg, 8, gm, bt, 1e-5, silu=True)
    torch.cuda.synchronize()
    blk = nat._block("gn", nat._GnArgs)[0]
    z2 = torch.empty_like(z1)
    rc = L.atk_group_norm_fwd(xg.data_ptr(), gm.data_ptr(), bt.data_ptr(), z2.data_ptr(), 2, 32, 256, 8,
                              ctypes.c_float(1e-5), 1, nat._DTYPE_CODE[xg.dtype], nat._DTYPE_CODE[gm.dtype],
                              blk.variant, blk.workspace, blk.workspace_bytes, nat._stream(xg))
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(z1, z2)
    # prepacked conv: the block's own fields replayed through the positional entry point
    xc, wc, bc = _conv_case(dev, (1, 64, 4, 16, 16), torch.bfloat16, 12)
    vi = _mfma_variant(nat, torch.bfloat16)
    c1 = nat.conv3d(xc, wc, bc, 1, 1, 1, variant=vi)
    torch.cuda.synchronize()
    a = nat._block("conv", nat._ConvArgs)[0]
    c2 = torch.empty_like(c1)
    geom = [getattr(a, f) for f in nat._CONV_GEOM_FIELDS]
    rc = L.atk_conv_fwd_prepacked(xc.data_ptr(), a.packed, a.packed_bytes, bc.data_ptr(), c2.data_ptr(), *geom,
                                  a.dtype, a.variant, a.workspace, a.workspace_bytes, nat._stream(xc))
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(c1, c2)
    assert O.max_rel_err(c1.cpu(), O.conv3d(xc.cpu(), wc.cpu(), bc.cpu(), 1, 1, 1)) <= 1e-2


def test_conv_plans_follow_shape_dtype_and_arguments(dev):
    """Alternating shapes, dtypes and argument spellings (ints, tuples, lists -- the last not
    memoised) through one thread's conv block: each result equals its first computation."""
    nat = _nat()
    cases = []
    for shape, dtype, pad in [((1, 64, 4, 16, 16), torch.bfloat16, 1), ((1, 64, 6, 8, 8), torch.bfloat16, (1, 1, 1)),
                              ((1, 64, 4, 16, 16), torch.float16, [1, 1, 1]), ((2, 64, 4, 8, 8), torch.float32, 1)]:
        x, w, b = _conv_case(dev, shape, dtype, seed=sum(shape))
        vi = _mfma_variant(nat, dtype)
        first = nat.conv3d(x, w, b, 1, pad, 1, variant=vi).clone()
        cases.append((x, w, b, pad, vi, first))
    for _ in range(2):
        for x, w, b, pad, vi, first in cases:
            assert torch.equal(nat.conv3d(x, w, b, 1, pad, 1, variant=vi), first)
    torch.cuda.synchronize()


def test_threads_calling_at_once_match_single_threaded(dev):
    """Four threads, each alternating two conv shapes, a GroupNorm and a dwconv1d, 25 rounds
    each: every result equals the single-threaded one (each thread fills its own argument
    blocks; the calls share the current stream, which orders them)."""
    nat = _nat()
    convs = [_conv_case(dev, s, torch.bfloat16, seed=i) for i, s in enumerate([(1, 64, 4, 16, 16), (1, 64, 6, 8, 8)])]
    vi = _mfma_variant(nat, torch.bfloat16)
    g = torch.Generator().manual_seed(5)
    xg = torch.randn(2, 32, 16, 16, generator=g).to(torch.bfloat16).to(dev)
    xd = torch.randn(2, 8, 500, generator=g).to(torch.bfloat16).to(dev)
    wd = torch.randn(8, 3, generator=g).to(torch.bfloat16).to(dev)
    refs = [nat.conv3d(x, w, b, 1, 1, 1, variant=vi).clone() for x, w, b in convs]
    ref_g = nat.group_norm(xg, 8, None, None, 1e-5).clone()
    ref_d = nat.dwconv1d(xd, wd, None, 1, 500).clone()
    torch.cuda.synchronize()
    errors = []

    def work(k):
        try:
            for it in range(25):
                j = (it + k) % 2
                x, w, b = convs[j]
                outs = [(nat.conv3d(x, w, b, 1, 1, 1, variant=vi), refs[j]),
                        (nat.group_norm(xg, 8, None, None, 1e-5), ref_g),
                        (nat.dwconv1d(xd, wd, None, 1, 500), ref_d)]
                torch.cuda.synchronize()
                for got, want in outs:
                    if not torch.equal(got, want):
                        errors.append((k, it))
        except Exception as exc:  # surfaced below
            errors.append(repr(exc))

    threads = [threading.Thread(target=work, args=(k,)) for k in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors[:5]
