"""GPU parity of the GroupNorm (+ fused SiLU) kernels (C ABI atk_group_norm_fwd) against
the float64 oracle, every variant.  Bars: fp32 <= 1e-5 max-abs-rel, fp16/bf16 <= 1e-2."""
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


def _inputs(shape, dtype, seed=0, affine=True, pdtype=None):
    g = torch.Generator().manual_seed(seed)
    C = shape[1]
    mu = torch.rand(C, generator=g) * 4 - 2          # per-channel means in U(-2, 2)
    x = torch.randn(*shape, generator=g) + mu.view(1, C, *([1] * (len(shape) - 2)))
    gamma = 1 + 0.1 * torch.randn(C, generator=g)
    beta = 0.1 * torch.randn(C, generator=g)
    pdtype = pdtype or dtype
    if not affine:
        return x.to(dtype), None, None
    return x.to(dtype), gamma.to(pdtype), beta.to(pdtype)


def _check(y, x, G, gamma, beta, eps, silu=False, what=""):
    ref = O.group_norm(x, G, gamma, beta, eps, silu=silu)
    err = O.max_rel_err(y, ref)
    assert err <= BAR[y.dtype], f"{what} max_rel_err {err:.3g} > {BAR[y.dtype]}"
    return err


SHAPES = [
    ((2, 64, 8, 8), 8),           # one small slice per group
    ((1, 32, 128, 128), 2),       # groups of 262144 elements: several slices per group
    ((2, 12, 5, 7, 8), 3),        # 3-D spatial
    ((3, 10, 24), 5),             # 1-D spatial
]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("shape_g", SHAPES, ids=lambda s: "x".join(map(str, s[0])) + f"_g{s[1]}")
def test_group_norm_all_variants(dev, shape_g, dtype):
    shape, G = shape_g
    nat = _native()
    x, gm, bt = _inputs(shape, dtype, seed=len(shape) + G)
    xd, gd, bd = x.to(dev), gm.to(dev), bt.to(dev)
    ran = 0
    for vi, name in enumerate(nat.variants(nat.OP_GROUP_NORM)):
        for silu in (False, True):
            try:
                y = nat.group_norm(xd, G, gd, bd, 1e-5, silu=silu, variant=vi)
            except nat.Unsupported:
                assert name != "twopass", "the two-pass variant must accept every shape"
                continue
            torch.cuda.synchronize()
            _check(y.cpu(), x, G, gm, bt, 1e-5, silu=silu, what=f"{name} silu={silu}")
            ran += 1
    assert ran >= 2
    assert not nat.group_norm_barrier_error(dev)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_group_norm_odd_spatial_and_2d(dev, dtype):
    """S not a multiple of the vector width, and [N, C] input (S = 1): only the two-pass
    kernel takes them; the register-resident variants decline."""
    nat = _native()
    names = nat.variants(nat.OP_GROUP_NORM)
    for shape, G in (((2, 6, 7, 7), 3), ((4, 16), 4)):
        x, gm, bt = _inputs(shape, dtype, seed=5)
        for vi, name in enumerate(names):
            if name == "twopass":
                y = nat.group_norm(x.to(dev), G, gm.to(dev), bt.to(dev), 1e-5, variant=vi)
                torch.cuda.synchronize()
                _check(y.cpu(), x, G, gm, bt, 1e-5)
            else:
                with pytest.raises(nat.Unsupported):
                    nat.group_norm(x.to(dev), G, gm.to(dev), bt.to(dev), 1e-5, variant=vi)


def test_group_norm_non_affine_and_mixed_param_dtype(dev):
    nat = _native()
    x, _, _ = _inputs((2, 32, 16, 16), torch.float16, seed=9, affine=False)
    y = nat.group_norm(x.to(dev), 8, None, None, 1e-6)
    _check(y.cpu(), x, 8, None, None, 1e-6)
    x, gm, bt = _inputs((2, 32, 16, 16), torch.bfloat16, seed=10, pdtype=torch.float32)
    y = nat.group_norm(x.to(dev), 8, gm.to(dev), bt.to(dev), 1e-5, silu=True)
    _check(y.cpu(), x, 8, gm, bt, 1e-5, silu=True)


def test_group_norm_misaligned_pointer(dev):
    nat = _native()
    x, gm, bt = _inputs((2, 16, 8, 8), torch.float16, seed=11)
    buf = torch.zeros(x.numel() + 1, dtype=x.dtype)
    buf[1:] = x.flatten()
    xv = buf.to(dev)[1:].view(x.shape)
    names = nat.variants(nat.OP_GROUP_NORM)
    y = nat.group_norm(xv, 4, gm.to(dev), bt.to(dev), 1e-5, variant=names.index("twopass"))
    _check(y.cpu(), x, 4, gm, bt, 1e-5)
    with pytest.raises(nat.Unsupported):
        nat.group_norm(xv, 4, gm.to(dev), bt.to(dev), 1e-5, variant=names.index("res_nt1024_v8"))


def test_group_norm_repeated_calls_keep_slots_consistent(dev):
    """Register-resident variants reuse the workspace slots: many calls in a row, different
    slice counts, all correct, and no workgroup ever had to stand in for another."""
    nat = _native()
    names = nat.variants(nat.OP_GROUP_NORM)
    x, gm, bt = _inputs((1, 32, 128, 128), torch.bfloat16, seed=12)
    xd, gd, bd = x.to(dev), gm.to(dev), bt.to(dev)
    ref = O.group_norm(x, 2, gm, bt, 1e-5)
    for _ in range(5):
        for name in ("res_nt256_v8", "res_nt1024_v8", "res_nt512_v8"):
            y = nat.group_norm(xd, 2, gd, bd, 1e-5, variant=names.index(name))
            torch.cuda.synchronize()
            assert O.max_rel_err(y.cpu(), ref) <= 1e-2
    assert not nat.group_norm_barrier_error(dev)


def test_group_norm_standin_path_is_bit_identical(dev, monkeypatch):
    """With a zero wait, workgroups compute every slice that is not yet published
    themselves.  The statistics must come out bit-identical to the normal path (same
    arithmetic in the same order), so the outputs are equal byte for byte."""
    nat = _native()
    names = nat.variants(nat.OP_GROUP_NORM)
    x, gm, bt = _inputs((1, 64, 32, 32, 16), torch.bfloat16, seed=13)   # 32 groups x 32768
    xd, gd, bd = x.to(dev), gm.to(dev), bt.to(dev)
    ref = O.group_norm(x, 32, gm, bt, 1e-5, silu=True)
    for name in ("res_nt256_v4", "res_nt256_v8"):
        vi = names.index(name)
        y0 = nat.group_norm(xd, 32, gd, bd, 1e-5, silu=True, variant=vi)
        torch.cuda.synchronize()
        assert not nat.group_norm_barrier_error(dev)
        monkeypatch.setenv("ATK_GN_WAIT_US", "0")
        for _ in range(3):
            y1 = nat.group_norm(xd, 32, gd, bd, 1e-5, silu=True, variant=vi)
            torch.cuda.synchronize()
            assert torch.equal(y0.view(torch.int16), y1.view(torch.int16)), name
        monkeypatch.delenv("ATK_GN_WAIT_US")
        assert O.max_rel_err(y1.cpu(), ref) <= 1e-2
        nat.group_norm_clear_diag(dev)


def test_group_norm_graph_replay(dev):
    """Captured in a HIP graph and replayed with new inputs copied in between replays
    (eager work and synchronisation between them): every replay matches the oracle --
    each launch empties its slots, so nothing carries over to the next replay."""
    nat = _native()
    names = nat.variants(nat.OP_GROUP_NORM)
    shape, G = (1, 64, 32, 32, 16), 32
    data = [_inputs(shape, torch.bfloat16, seed=40 + i) for i in range(3)]
    gm, bt = data[0][1], data[0][2]
    gd, bd = gm.to(dev), bt.to(dev)
    static_x = data[0][0].to(dev)
    for name in ("res_nt256_v4", "res_nt512_v8", "twopass"):
        vi = names.index(name)
        out = torch.empty_like(static_x)
        nat.group_norm(static_x, G, gd, bd, 1e-5, silu=True, variant=vi, out=out)  # allocates workspace
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            nat.group_norm(static_x, G, gd, bd, 1e-5, silu=True, variant=vi, out=out)
        for _ in range(2):
            for x, _, _ in data:
                static_x.copy_(x.to(dev))
                torch.cuda.synchronize()
                graph.replay()
                torch.cuda.synchronize()
                ref = O.group_norm(x, G, gm, bt, 1e-5, silu=True)
                assert O.max_rel_err(out.cpu(), ref) <= 1e-2, name
    assert not nat.group_norm_barrier_error(dev)


CONFIG3 = [((8, 512, 64, 64), 32, 1e-5), ((1, 512, 16, 64, 64), 32, 1e-5),
           ((1, 256, 8, 64, 64), 32, 1e-6)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("cfg", CONFIG3, ids=["c3_nchw", "c3_ncdhw", "c5_gn"])
def test_group_norm_config_full_size(dev, cfg, dtype):
    """BASELINE configs 3 and 5 (GroupNorm part) at full size, plain and fused SiLU, every
    variant that accepts the shape."""
    shape, G, eps = cfg
    nat = _native()
    x, gm, bt = _inputs(shape, dtype, seed=1003)
    xd, gd, bd = x.to(dev), gm.to(dev), bt.to(dev)
    for silu in (False, True):
        ref = O.group_norm(x, G, gm, bt, eps, silu=silu)
        for vi, name in enumerate(nat.variants(nat.OP_GROUP_NORM)):
            try:
                y = nat.group_norm(xd, G, gd, bd, eps, silu=silu, variant=vi)
            except nat.Unsupported:
                continue
            torch.cuda.synchronize()
            err = O.max_rel_err(y.cpu(), ref)
            assert err <= 1e-2, f"{name} silu={silu}: {err:.3g}"
    assert not nat.group_norm_barrier_error(dev)


def test_group_norm_workspace_shared_across_shapes(dev):
    """Regression: a shape with few groups and many slices writes many partials into the
    shared workspace; a following multi-slice call on a shape with many groups must not
    mistake those for its own slots (slots carry a per-launch tag)."""
    nat = _native()
    names = nat.variants(nat.OP_GROUP_NORM)
    xa, ga, ba = _inputs((8, 256, 64, 64), torch.float16, seed=21)    # 256 groups of 32768
    xb, gb, bb = _inputs((1, 64, 64, 64, 16), torch.float16, seed=22)  # 32 groups of 131072
    ref_a = O.group_norm(xa, 32, ga, ba, 1e-5)
    ref_b = O.group_norm(xb, 32, gb, bb, 1e-5)
    xa, ga, ba, xb, gb, bb = (t.to(dev) for t in (xa, ga, ba, xb, gb, bb))
    for _ in range(2):
        for name in ("res_nt256_v8", "twopass", "res_nt256_v16"):
            yb = nat.group_norm(xb, 32, gb, bb, 1e-5, variant=names.index(name))
            ya = nat.group_norm(xa, 32, ga, ba, 1e-5, variant=names.index("res_nt256_v8"))
            torch.cuda.synchronize()
            assert O.max_rel_err(yb.cpu(), ref_b) <= 1e-2
            assert O.max_rel_err(ya.cpu(), ref_a) <= 1e-2
    assert not nat.group_norm_barrier_error(dev)


# ---------------------------------------------------------------------------
# backward (atk_group_norm_bwd) against the float64 oracle
# ---------------------------------------------------------------------------
# dgamma / dbeta are fp32 sums of exact products: tighter than the 16-bit output bar
BWD_BAR_P = {torch.float32: 1e-5, torch.float16: 1e-4, torch.bfloat16: 1e-4}

BWD_SHAPES = [
    ((2, 64, 8, 8), 8, True),
    ((1, 32, 128, 128), 2, True),     # large groups
    ((2, 12, 4, 6, 8), 3, False),     # 3-D spatial, no affine
    ((3, 10, 24), 5, True),           # 1-D spatial
    ((8, 512, 16, 16), 32, True),     # C3-like channel count
    # register-resident backward (spatial size a multiple of 64 vectors, group <= 8192 vectors)
    ((4, 64, 32, 32), 8, True),
    ((3, 96, 16, 32), 6, False),      # three samples per group counter, no affine
    ((1, 32, 8, 64, 64), 4, True),    # one sample, groups of the largest resident size (16-bit)
]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("case", BWD_SHAPES, ids=lambda s: "x".join(map(str, s[0])) + f"_g{s[1]}")
def test_group_norm_backward_native(dev, case, dtype):
    shape, G, affine = case
    nat = _native()
    x, gm, _ = _inputs(shape, dtype, seed=len(shape) + G + 100, affine=affine)
    dy = torch.randn(*shape, generator=torch.Generator().manual_seed(G)).to(dtype)
    dx, dg, db = nat.group_norm_backward(dy.to(dev), x.to(dev), G, None if gm is None else gm.to(dev),
                                         1e-5, (True, True, True))
    torch.cuda.synchronize()
    rdx, rdg, rdb = O.group_norm_bwd(x, G, gm, dy, 1e-5)
    assert dx.dtype == dtype
    assert O.max_rel_err(dx.cpu(), rdx) <= BAR[dtype], O.max_rel_err(dx.cpu(), rdx)
    assert O.max_rel_err(dg.cpu(), rdg) <= BWD_BAR_P[dtype], O.max_rel_err(dg.cpu(), rdg)
    assert O.max_rel_err(db.cpu(), rdb) <= BWD_BAR_P[dtype], O.max_rel_err(db.cpu(), rdb)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_group_norm_autograd_through_patched_group_norm(dev, dtype):
    """Training path: the patched F.group_norm with requires_grad inputs runs the native
    forward and the native backward; gradients match the oracle.  A spatial size that is
    not a multiple of 16 bytes takes the torch-op backward and must agree too."""
    import torch.nn.functional as F
    import amd_tuned_torch  # noqa: F401
    for shape, G in (((2, 16, 8, 8), 4), ((2, 8, 3, 5), 2)):
        x, gm, bt = _inputs(shape, dtype, seed=7 + G)
        xd = x.to(dev).requires_grad_(True)
        gd, bd = gm.to(dev).requires_grad_(True), bt.to(dev).requires_grad_(True)
        y = F.group_norm(xd, G, gd, bd, 1e-5)
        dy = torch.randn(*shape, generator=torch.Generator().manual_seed(3)).to(dtype)
        gx, gg, gb = torch.autograd.grad(y, (xd, gd, bd), dy.to(dev))
        rdx, rdg, rdb = O.group_norm_bwd(x, G, gm, dy, 1e-5)
        assert O.max_rel_err(gx.cpu(), rdx) <= BAR[dtype]
        assert O.max_rel_err(gg.cpu(), rdg) <= BAR[dtype]
        assert O.max_rel_err(gb.cpu(), rdb) <= BAR[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_group_norm_autograd_channels_last(dev, dtype):
    """Channels-last (NHWC / NDHWC) input through the patched F.group_norm with gradients:
    x and dy reach the native channels-last backward, dx comes back channels-last; every
    gradient matches the oracle."""
    import torch.nn.functional as F
    import amd_tuned_torch  # noqa: F401
    for shape, G, fmt in (((2, 64, 8, 8), 8, torch.channels_last),
                          ((1, 32, 4, 8, 8), 4, torch.channels_last_3d)):
        x, gm, bt = _inputs(shape, dtype, seed=11 + G)
        xd = x.to(dev).contiguous(memory_format=fmt).requires_grad_(True)
        gd, bd = gm.to(dev).requires_grad_(True), bt.to(dev).requires_grad_(True)
        y = F.group_norm(xd, G, gd, bd, 1e-5)
        dy = torch.randn(*shape, generator=torch.Generator().manual_seed(5)).to(dtype)
        gx, gg, gb = torch.autograd.grad(y, (xd, gd, bd), dy.to(dev).contiguous(memory_format=fmt))
        assert gx.is_contiguous(memory_format=fmt)
        rdx, rdg, rdb = O.group_norm_bwd(x, G, gm, dy, 1e-5)
        assert O.max_rel_err(gx.cpu().contiguous(), rdx) <= BAR[dtype]
        assert O.max_rel_err(gg.cpu(), rdg) <= BAR[dtype]
        assert O.max_rel_err(gb.cpu(), rdb) <= BAR[dtype]


@pytest.mark.parametrize("needs", [(True, False, False), (False, True, True), (True, True, False)],
                         ids=["dx_only", "params_only", "dx_dgamma"])
def test_group_norm_backward_resident_subsets(dev, needs):
    """The register-resident backward with some gradients not asked for; two calls in a row
    (the per-group counters must be left zero by the first)."""
    nat = _native()
    shape, G = (2, 64, 16, 64), 8
    x, gm, _ = _inputs(shape, torch.bfloat16, seed=77)
    dy = torch.randn(*shape, generator=torch.Generator().manual_seed(78)).to(torch.bfloat16)
    rdx, rdg, rdb = O.group_norm_bwd(x, G, gm, dy, 1e-5)
    for _ in range(2):
        dx, dg, db = nat.group_norm_backward(dy.to(dev), x.to(dev), G, gm.to(dev), 1e-5, needs)
        torch.cuda.synchronize()
        for got, ref, want, bar in ((dx, rdx, needs[0], BAR[torch.bfloat16]),
                                    (dg, rdg, needs[1], BWD_BAR_P[torch.bfloat16]),
                                    (db, rdb, needs[2], BWD_BAR_P[torch.bfloat16])):
            assert (got is not None) == want
            if want:
                assert O.max_rel_err(got.cpu(), ref) <= bar


def test_group_norm_backward_c3a_full_size(dev):
    """C3's NCHW shape at full size, bf16 (the register-resident backward): every gradient
    element against the oracle."""
    nat = _native()
    shape, G = (8, 512, 64, 64), 32
    x, gm, _ = _inputs(shape, torch.bfloat16, seed=3005)
    dy = torch.randn(*shape, generator=torch.Generator().manual_seed(3006)).to(torch.bfloat16)
    dx, dg, db = nat.group_norm_backward(dy.to(dev), x.to(dev), G, gm.to(dev), 1e-5, (True, True, True))
    torch.cuda.synchronize()
    rdx, rdg, rdb = O.group_norm_bwd(x, G, gm, dy, 1e-5)
    assert O.max_rel_err(dx.cpu(), rdx) <= BAR[torch.bfloat16]
    assert O.max_rel_err(dg.cpu(), rdg) <= BWD_BAR_P[torch.bfloat16]
    assert O.max_rel_err(db.cpu(), rdb) <= BWD_BAR_P[torch.bfloat16]


def test_group_norm_backward_c3_full_size(dev):
    """C3's NCDHW shape at full size, bf16: every gradient element against the oracle."""
    nat = _native()
    shape, G = (1, 512, 16, 64, 64), 32
    x, gm, _ = _inputs(shape, torch.bfloat16, seed=3003)
    dy = torch.randn(*shape, generator=torch.Generator().manual_seed(3004)).to(torch.bfloat16)
    dx, dg, db = nat.group_norm_backward(dy.to(dev), x.to(dev), G, gm.to(dev), 1e-5, (True, True, True))
    torch.cuda.synchronize()
    rdx, rdg, rdb = O.group_norm_bwd(x, G, gm, dy, 1e-5)
    assert O.max_rel_err(dx.cpu(), rdx) <= BAR[torch.bfloat16]
    assert O.max_rel_err(dg.cpu(), rdg) <= BWD_BAR_P[torch.bfloat16]
    assert O.max_rel_err(db.cpu(), rdb) <= BWD_BAR_P[torch.bfloat16]


# ---------------------------------------------------------------------------
# channels-last forward (atk_group_norm_cl_fwd)
# ---------------------------------------------------------------------------
CL_SHAPES = [
    ((2, 64, 8, 8), 8),
    ((8, 512, 16, 16), 32),         # C3-like channels, NHWC
    ((1, 256, 4, 16, 16), 32),      # C5-like channels, NDHWC
    ((3, 32, 7, 5), 4),             # odd spatial sizes
]


CL_BWD_SHAPES = CL_SHAPES + [
    ((1, 64, 1, 2048), 4),          # one long row: 32 chunks of 64 positions
    ((2, 128, 3, 40, 40), 16),      # NDHWC, chunk boundaries inside rows
]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("shape_g", CL_BWD_SHAPES, ids=lambda s: "x".join(map(str, s[0])) + f"_g{s[1]}")
def test_group_norm_channels_last_backward(dev, shape_g, dtype):
    """atk_group_norm_cl_bwd on channels-last x and dy against the float64 oracle (which
    reads the same values in NC[S] order): dx in the input's memory format, dgamma, dbeta;
    also without affine weights and with only the parameter gradients asked for."""
    shape, G = shape_g
    nat = _native()
    x, gm, _ = _inputs(shape, dtype, seed=len(shape) + G + 300)
    dy = torch.randn(*shape, generator=torch.Generator().manual_seed(G + 7)).to(dtype)
    fmt = torch.channels_last if len(shape) == 4 else torch.channels_last_3d
    xd, dyd = x.to(dev).contiguous(memory_format=fmt), dy.to(dev).contiguous(memory_format=fmt)
    for weight in (gm, None):
        dx, dg, db = nat.group_norm_cl_backward(dyd, xd, G, None if weight is None else weight.to(dev), 1e-5)
        torch.cuda.synchronize()
        assert dx.is_contiguous(memory_format=fmt) and dx.dtype == dtype
        rdx, rdg, rdb = O.group_norm_bwd(x, G, weight, dy, 1e-5)
        assert O.max_rel_err(dx.cpu().contiguous(), rdx) <= BAR[dtype], O.max_rel_err(dx.cpu().contiguous(), rdx)
        assert O.max_rel_err(dg.cpu(), rdg) <= BWD_BAR_P[dtype], O.max_rel_err(dg.cpu(), rdg)
        assert O.max_rel_err(db.cpu(), rdb) <= BWD_BAR_P[dtype], O.max_rel_err(db.cpu(), rdb)
    dx2, dg2, db2 = nat.group_norm_cl_backward(dyd, xd, G, gm.to(dev), 1e-5, (False, True, True))
    assert dx2 is None and torch.equal(dg2.cpu(), nat.group_norm_cl_backward(dyd, xd, G, gm.to(dev), 1e-5)[1].cpu())


@pytest.mark.parametrize("mode", ["16", "0"])
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("shape_g", CL_BWD_SHAPES + [((2, 256, 100, 130), 32), ((1, 256, 31, 256), 32)],
                         ids=lambda s: "x".join(map(str, s[0])) + f"_g{s[1]}")
def test_group_norm_channels_last_backward_resident(dev, shape_g, dtype, mode, monkeypatch):
    """The channels-last backward forced onto the register-resident kernel (and, "0", onto
    the three kernels) wherever it fits: dx, dgamma, dbeta against the float64 oracle, with
    and without affine weights; repeats are bit-identical and no record was computed by a
    stand-in.  (2,256,100,130) has 51 chunks per sample (two-level), (1,256,31,256) 31 of 32
    groups (direct)."""
    shape, G = shape_g
    nat = _native()
    monkeypatch.setenv("ATK_GN_CL_RESIDENT", mode)
    x, gm, _ = _inputs(shape, dtype, seed=len(shape) + G + 900)
    dy = torch.randn(*shape, generator=torch.Generator().manual_seed(G + 17)).to(dtype)
    fmt = torch.channels_last if len(shape) == 4 else torch.channels_last_3d
    xd, dyd = x.to(dev).contiguous(memory_format=fmt), dy.to(dev).contiguous(memory_format=fmt)
    for weight in (gm, None):
        wd = None if weight is None else weight.to(dev)
        dx, dg, db = nat.group_norm_cl_backward(dyd, xd, G, wd, 1e-5)
        dx2, dg2, db2 = nat.group_norm_cl_backward(dyd, xd, G, wd, 1e-5)
        torch.cuda.synchronize()
        assert torch.equal(dx, dx2) and torch.equal(dg, dg2) and torch.equal(db, db2), "repeat differs"
        rdx, rdg, rdb = O.group_norm_bwd(x, G, weight, dy, 1e-5)
        assert O.max_rel_err(dx.cpu().contiguous(), rdx) <= BAR[dtype], O.max_rel_err(dx.cpu().contiguous(), rdx)
        assert O.max_rel_err(dg.cpu(), rdg) <= BWD_BAR_P[dtype], O.max_rel_err(dg.cpu(), rdg)
        assert O.max_rel_err(db.cpu(), rdb) <= BWD_BAR_P[dtype], O.max_rel_err(db.cpu(), rdb)
    dxn, dgn, dbn = nat.group_norm_cl_backward(dyd, xd, G, gm.to(dev), 1e-5, (False, True, True))
    assert dxn is None and torch.equal(dgn, nat.group_norm_cl_backward(dyd, xd, G, gm.to(dev), 1e-5)[1])
    assert not nat.group_norm_barrier_error(dev)


@pytest.mark.parametrize("shape", [(1, 256, 65, 256), (1, 256, 31, 256)], ids=["two_level", "direct"])
def test_group_norm_channels_last_backward_standin_and_replay(dev, shape, monkeypatch):
    """Resident channels-last backward: with a zero wait (stand-ins for records not yet
    published) the outputs equal the normal path's byte for byte; captured in a HIP graph and
    replayed with new inputs copied in between, every replay equals an eager run."""
    nat = _native()
    G = 32
    monkeypatch.setenv("ATK_GN_CL_RESIDENT", "16")
    fmt = torch.channels_last
    data = []
    for i in range(3):
        x, gm, _ = _inputs(shape, torch.bfloat16, seed=950 + i)
        dy = torch.randn(*shape, generator=torch.Generator().manual_seed(960 + i)).to(torch.bfloat16)
        data.append((x.to(dev).contiguous(memory_format=fmt), dy.to(dev).contiguous(memory_format=fmt)))
    gd = _inputs(shape, torch.bfloat16, seed=950)[1].to(dev)
    ref = nat.group_norm_cl_backward(data[0][1], data[0][0], G, gd, 1e-5)
    torch.cuda.synchronize()
    assert not nat.group_norm_barrier_error(dev)
    monkeypatch.setenv("ATK_GN_WAIT_US", "0")
    for _ in range(2):
        got = nat.group_norm_cl_backward(data[0][1], data[0][0], G, gd, 1e-5)
        torch.cuda.synchronize()
        for a, b in zip(got, ref):
            assert torch.equal(a, b)
    monkeypatch.delenv("ATK_GN_WAIT_US")
    nat.group_norm_clear_diag(dev)
    xs, dys = data[0][0].clone(), data[0][1].clone()
    nat.group_norm_cl_backward(dys, xs, G, gd, 1e-5)   # workspace allocated before capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = nat.group_norm_cl_backward(dys, xs, G, gd, 1e-5)
    for rep in range(6):
        xs.copy_(data[rep % 3][0])
        dys.copy_(data[rep % 3][1])
        graph.replay()
        torch.cuda.synchronize()
        eager = nat.group_norm_cl_backward(dys, xs, G, gd, 1e-5)
        torch.cuda.synchronize()
        for a, b in zip(out, eager):
            assert torch.equal(a, b), f"replay {rep}"
    assert not nat.group_norm_barrier_error(dev)


def test_group_norm_channels_last_backward_c3_full_size(dev):
    """C3's NDHWC shape at full size, bf16, through the channels-last backward kernels:
    every gradient element against the oracle."""
    nat = _native()
    shape, G = (1, 512, 16, 64, 64), 32
    x, gm, _ = _inputs(shape, torch.bfloat16, seed=3103)
    dy = torch.randn(*shape, generator=torch.Generator().manual_seed(3104)).to(torch.bfloat16)
    fmt = torch.channels_last_3d
    dx, dg, db = nat.group_norm_cl_backward(dy.to(dev).contiguous(memory_format=fmt),
                                            x.to(dev).contiguous(memory_format=fmt), G, gm.to(dev), 1e-5)
    torch.cuda.synchronize()
    rdx, rdg, rdb = O.group_norm_bwd(x, G, gm, dy, 1e-5)
    assert O.max_rel_err(dx.cpu().contiguous(), rdx) <= BAR[torch.bfloat16]
    assert O.max_rel_err(dg.cpu(), rdg) <= BWD_BAR_P[torch.bfloat16]
    assert O.max_rel_err(db.cpu(), rdb) <= BWD_BAR_P[torch.bfloat16]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("shape_g", CL_SHAPES, ids=lambda s: "x".join(map(str, s[0])) + f"_g{s[1]}")
def test_group_norm_channels_last(dev, shape_g, dtype):
    shape, G = shape_g
    nat = _native()
    x, gm, bt = _inputs(shape, dtype, seed=len(shape) + G + 200)
    fmt = torch.channels_last if len(shape) == 4 else torch.channels_last_3d
    xd = x.to(dev).contiguous(memory_format=fmt)
    for silu in (False, True):
        y = nat.group_norm_cl(xd, G, gm.to(dev), bt.to(dev), 1e-5, silu=silu)
        torch.cuda.synchronize()
        assert y.is_contiguous(memory_format=fmt)
        _check(y.cpu().contiguous(), x, G, gm, bt, 1e-5, silu=silu, what=f"cl silu={silu}")


# (shape, G, ATK_GN_CL_RESIDENT): which register-resident configuration the channels-last
# forward takes ("0" = the three-kernel path).  With at least as many chunks per sample as
# groups, one workgroup per group merges that group's chunk records (two-level); with fewer,
# every workgroup merges all G x NCH records (direct, at most 1024).  (2,256,100,130) bf16 has
# 102 chunks of 128 positions per sample at 8 vectors per thread and 51 of 256 at 16 (both
# two-level, a partial last chunk); (1,256,31,256) at 16 has 31 chunks of 32 groups (direct,
# 992 records); (8,512,16,16) and (1,64,3,1000) are direct.  Those are the `rows` chunk shape
# (all channels of SC positions); where the groups tile 8 columns (128 bytes of a position)
# and C spans more, `blocks` chunks hold 8 columns of EPV * 64 positions and a workgroup
# merges only its block's groups, in one round ((1,64,3,1000) in 16-bit types has only 8
# columns and stays rows).
CL_RES_CASES = [
    ((2, 256, 100, 130), 32, "8"),
    ((2, 256, 100, 130), 32, "16"),
    ((2, 256, 100, 130), 32, "0"),
    ((1, 512, 4, 32, 64), 32, "16"),    # C3-like channels, NDHWC (fp32: two-level)
    ((1, 256, 31, 256), 32, "16"),      # 31 x 32 records: direct (16-bit)
    ((8, 512, 16, 16), 32, "8"),
    ((1, 64, 3, 1000), 4, "16"),         # one sample, 1 chunk per 1024 positions
]


@pytest.mark.parametrize("layout", ["rows", "blocks"])
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("case", CL_RES_CASES, ids=lambda c: "x".join(map(str, c[0])) + f"_g{c[1]}_r{c[2]}")
def test_group_norm_channels_last_resident(dev, case, dtype, layout, monkeypatch):
    """The channels-last forward in each register-resident configuration and chunk shape (and
    the three-kernel path) against the oracle, with and without SiLU and affine parameters;
    repeated calls are bit-identical (the slot epoch advances between them) and no launch
    fell back to computing another workgroup's statistics."""
    shape, G, mode = case
    if mode == "0" and layout == "blocks":
        pytest.skip("the three-kernel path has no chunk shape")
    nat = _native()
    monkeypatch.setenv("ATK_GN_CL_RESIDENT", mode)
    monkeypatch.setenv("ATK_GN_CL_LAYOUT", layout)
    fmt = torch.channels_last if len(shape) == 4 else torch.channels_last_3d
    for affine in (True, False):
        x, gm, bt = _inputs(shape, dtype, seed=len(shape) + G + int(mode) + 500, affine=affine)
        xd = x.to(dev).contiguous(memory_format=fmt)
        gd = gm.to(dev) if gm is not None else None
        bd = bt.to(dev) if bt is not None else None
        for silu in (False, True):
            y = nat.group_norm_cl(xd, G, gd, bd, 1e-5, silu=silu)
            y2 = nat.group_norm_cl(xd, G, gd, bd, 1e-5, silu=silu)
            torch.cuda.synchronize()
            assert y.is_contiguous(memory_format=fmt)
            assert torch.equal(y, y2), f"repeat differs (mode {mode}, silu={silu})"
            _check(y.cpu().contiguous(), x, G, gm, bt, 1e-5, silu=silu,
                   what=f"cl resident={mode} silu={silu} affine={affine}")
    assert not nat.group_norm_barrier_error(dev)


@pytest.mark.parametrize("layout", ["rows", "blocks"])
@pytest.mark.parametrize("shape,mode", [((1, 256, 65, 128), "8"), ((1, 256, 31, 256), "16")],
                         ids=["two_level", "direct"])
def test_group_norm_channels_last_standin_bit_identical(dev, shape, mode, layout, monkeypatch):
    """With a zero wait, workgroups compute every chunk record (and, two-level, every group
    result) that is not yet published themselves; the outputs must equal the normal path's
    byte for byte.  Rows: 65 chunks x 32 groups at 8 vectors per thread (two-level); 31 x 32 at
    16 (direct).  Blocks: 4 channel blocks of 8 groups, 17 / 8 chunks each."""
    nat = _native()
    G = 32
    monkeypatch.setenv("ATK_GN_CL_RESIDENT", mode)
    monkeypatch.setenv("ATK_GN_CL_LAYOUT", layout)
    x, gm, bt = _inputs(shape, torch.bfloat16, seed=611)
    xd = x.to(dev).contiguous(memory_format=torch.channels_last)
    gd, bd = gm.to(dev), bt.to(dev)
    y0 = nat.group_norm_cl(xd, G, gd, bd, 1e-5, silu=True)
    torch.cuda.synchronize()
    assert not nat.group_norm_barrier_error(dev)
    monkeypatch.setenv("ATK_GN_WAIT_US", "0")
    for _ in range(3):
        y1 = nat.group_norm_cl(xd, G, gd, bd, 1e-5, silu=True)
        torch.cuda.synchronize()
        assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))
    monkeypatch.delenv("ATK_GN_WAIT_US")
    nat.group_norm_clear_diag(dev)
    _check(y1.cpu().contiguous(), x, G, gm, bt, 1e-5, silu=True, what="cl stand-in")


@pytest.mark.parametrize("layout", ["rows", "blocks"])
@pytest.mark.parametrize("mode", ["8", "16"])
def test_group_norm_channels_last_graph_replay(dev, mode, layout, monkeypatch):
    """The resident channels-last forward captured in a HIP graph and replayed with new
    inputs copied in between (eager work and synchronisation between replays): every replay
    matches the eager result bit for bit -- the slot epoch lives in device memory, so a
    replay never accepts a slot written by the previous one."""
    nat = _native()
    shape, G = (2, 256, 100, 130), 32
    monkeypatch.setenv("ATK_GN_CL_RESIDENT", mode)
    monkeypatch.setenv("ATK_GN_CL_LAYOUT", layout)
    data = [_inputs(shape, torch.bfloat16, seed=70 + i) for i in range(3)]
    gd, bd = data[0][1].to(dev), data[0][2].to(dev)
    xs = data[0][0].to(dev).contiguous(memory_format=torch.channels_last)
    out = torch.empty_like(xs)
    nat.group_norm_cl(xs, G, gd, bd, 1e-5, out=out)   # workspace allocated before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        nat.group_norm_cl(xs, G, gd, bd, 1e-5, out=out)
    for rep in range(6):
        x = data[rep % 3][0]
        xs.copy_(x.to(dev).contiguous(memory_format=torch.channels_last))
        g.replay()
        torch.cuda.synchronize()
        eager = nat.group_norm_cl(xs, G, gd, bd, 1e-5)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep}"
    _check(out.cpu().contiguous(), data[5 % 3][0], G, data[0][1], data[0][2], 1e-5, what="cl graph replay")
    assert not nat.group_norm_barrier_error(dev)


@pytest.mark.parametrize("silu", [False, True])
@pytest.mark.parametrize("shape", [(8, 512, 64, 64), (1, 512, 16, 64, 64)], ids=["c3a_nhwc", "c3b_ndhwc"])
def test_group_norm_channels_last_c3_full_size(dev, shape, silu):
    """C3's shapes in channels-last memory at full size, bf16, on the library's own choice of
    kernel and chunk shape: every element against the float64 oracle; a repeat is
    bit-identical and no statistics were computed by a stand-in."""
    nat = _native()
    G = 32
    x, gm, bt = _inputs(shape, torch.bfloat16, seed=3200 + len(shape))
    fmt = torch.channels_last if len(shape) == 4 else torch.channels_last_3d
    xd = x.to(dev).contiguous(memory_format=fmt)
    y = nat.group_norm_cl(xd, G, gm.to(dev), bt.to(dev), 1e-5, silu=silu)
    y2 = nat.group_norm_cl(xd, G, gm.to(dev), bt.to(dev), 1e-5, silu=silu)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    assert not nat.group_norm_barrier_error(dev)
    _check(y.cpu().contiguous(), x, G, gm, bt, 1e-5, silu=silu, what=f"cl full size {shape}")


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_group_norm_channels_last_through_patched_api(dev, dtype):
    """F.group_norm and conv_fusion_ops.group_norm_silu on channels-last tensors take the
    native channels-last kernel (or stock, whichever the contest keeps) and match the oracle."""
    import torch.nn.functional as F
    import amd_tuned_torch  # noqa: F401
    from amd_tuned_torch import conv_fusion_ops
    shape, G = (4, 128, 12, 12), 16
    x, gm, bt = _inputs(shape, dtype, seed=303)
    xd = x.to(dev).contiguous(memory_format=torch.channels_last)
    y = F.group_norm(xd, G, gm.to(dev), bt.to(dev), 1e-5)
    _check(y.cpu().contiguous(), x, G, gm, bt, 1e-5, what="F.group_norm channels-last")
    y2 = conv_fusion_ops.group_norm_silu(xd, G, gm.to(dev), bt.to(dev), 1e-5)
    _check(y2.cpu().contiguous(), x, G, gm, bt, 1e-5, silu=True, what="group_norm_silu channels-last")
