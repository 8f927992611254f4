"""torch.library custom ops of the package (amd_tuned_torch/compile_ops.py and
depthwise_conv1d_ops.py), on the CPU: their fake (meta) kernels give the output shapes and
dtypes Dynamo traces with, without touching the native library.  Known answers follow the
reference's own fake-shape tests (tests/test_compile_ops.py:90-130,
tests/test_depthwise_conv1d_ops.py:84-127)."""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch._subclasses.fake_tensor import FakeTensorMode

import amd_tuned_torch  # noqa: F401  (registers the ops)
from amd_tuned_torch import compile_ops, depthwise_conv1d_ops  # noqa: F401

ops = torch.ops.amd_tuned_torch


def test_group_norm_fake_shape():
    with FakeTensorMode():
        x = torch.randn(2, 4, 3, 3)
        out = ops.group_norm(x, 2, None, None, 1e-5)
    assert out.shape == x.shape and out.dtype == x.dtype


def test_conv2d_native_fake_shapes():
    with FakeTensorMode():
        x = torch.randn(1, 3, 8, 8)
        w = torch.randn(4, 3, 3, 3)
        same = ops.conv2d_native(x, w, None, [1, 1], [1, 1], [1, 1])
        strided = ops.conv2d_native(x, w, None, [2, 2], [1, 1], [1, 1])
    assert same.shape == (1, 4, 8, 8)
    expected = F.conv2d(torch.randn(1, 3, 8, 8), torch.randn(4, 3, 3, 3), stride=2, padding=1)
    assert strided.shape == expected.shape


def test_conv3d_native_fake_shape():
    with FakeTensorMode():
        x = torch.randn(1, 3, 4, 8, 8)
        w = torch.randn(4, 3, 3, 3, 3)
        out = ops.conv3d_native(x, w, None, [1, 1, 1], [1, 1, 1], [1, 1, 1])
    assert out.shape == (1, 4, 4, 8, 8)


def test_depthwise_conv1d_forward_fake_shapes():
    with FakeTensorMode():
        x = torch.randn(2, 4, 10)
        bhl = ops.depthwise_conv1d_forward(x, torch.randn(4, 3), torch.randn(4), 1, True)
        xl = torch.randn(2, 10, 4)
        blh = ops.depthwise_conv1d_forward(xl, torch.randn(3, 4), torch.randn(4), 0, False)
    assert bhl.shape == (2, 4, 10) and bhl.dtype == x.dtype
    assert blh.shape == (2, 8, 4) and blh.dtype == xl.dtype


def test_depthwise_conv1d_backward_fake_shapes_and_dtypes():
    """dbias takes dout's dtype, dweight the weight's, du the input's."""
    with FakeTensorMode():
        x = torch.randn(2, 4, 10, dtype=torch.float32)
        w = torch.randn(4, 3, dtype=torch.float16)
        b = torch.randn(4, dtype=torch.float16)
        dout = torch.randn(2, 4, 10, dtype=torch.float32)
        du, dweight, dbias = ops.depthwise_conv1d_backward(dout, x, w, b, 1, True)
    assert du.shape == x.shape and du.dtype == x.dtype
    assert dweight.shape == w.shape and dweight.dtype == w.dtype
    assert dbias.shape == b.shape and dbias.dtype == dout.dtype


# ---------------------------------------------------------------------------
# torch.compile routing of the patched API (fake cuda tensors: Dynamo traces without a GPU)
# ---------------------------------------------------------------------------
def _capture(fn, *args):
    """Compile fn with fullgraph=True (any graph break raises) and return the call targets
    of the one captured FX graph."""
    import torch._dynamo
    torch._dynamo.reset()
    graphs = []

    def backend(gm, example_inputs):
        graphs.append(gm)
        return gm.forward
    out = torch.compile(fn, backend=backend, fullgraph=True)(*args)
    assert len(graphs) == 1
    return out, [n.target for n in graphs[0].graph.nodes if n.op == "call_function"]


def _fake_cuda(*shapes, dtype=torch.bfloat16, requires_grad=False):
    with FakeTensorMode(allow_non_fake_inputs=True):
        out = [torch.empty(s, device="cuda", dtype=dtype) for s in shapes]
    return [t.requires_grad_(requires_grad) for t in out]


def test_compiled_patched_ops_are_custom_op_nodes():
    """Each patched entry point becomes one amd_tuned_torch node; no graph break, no Python
    dispatch (ctypes, the selector) in the graph."""
    x, w3, b3, g, b, x1, w1, b1, x2, w2 = _fake_cuda(
        (1, 8, 4, 8, 8), (8, 8, 3, 3, 3), (8,), (8,), (8,), (2, 16, 64), (16, 1, 3), (16,),
        (1, 8, 8, 8), (8, 8, 3, 3))

    def block(x, w3, b3, g, b, x1, w1, b1, x2, w2):
        y = F.conv3d(x, w3, b3, 1, 1)
        y = F.group_norm(y, 4, g, b, 1e-5)
        y = amd_tuned_torch.group_norm_silu(y, 4, g, b, 1e-5)
        z = F.conv1d(x1, w1, b1, padding=1, groups=16)
        u = F.conv2d(x2, w2, None, 1, 1)
        return y, z, u

    (y, z, u), targets = _capture(block, x, w3, b3, g, b, x1, w1, b1, x2, w2)
    assert y.shape == x.shape and z.shape == x1.shape and u.shape == x2.shape
    names = [str(t) for t in targets]
    for op in ("conv3d_native", "group_norm", "group_norm_silu", "depthwise_conv1d_forward",
               "conv2d_native"):
        assert "amd_tuned_torch.%s" % op in names, names


def test_compiled_routes_leave_ineligible_calls_to_stock():
    """Grouped conv, 1x1 pointwise conv2d and string padding trace as stock aten calls."""
    x, w_grp, w_pt = _fake_cuda((1, 8, 8, 8), (8, 4, 3, 3), (8, 8, 1, 1))

    def f(x, w_grp, w_pt):
        return F.conv2d(x, w_grp, None, 1, 1, 1, 2), F.conv2d(x, w_pt), F.conv2d(x, w_pt, padding="same")

    _, targets = _capture(f, x, w_grp, w_pt)
    assert not any("amd_tuned_torch" in str(t) for t in targets), targets


def test_compiled_routes_with_gradients_keep_custom_ops():
    """With parameters that require grad the same nodes appear (their autograd formulas are
    registered); GroupNorm+SiLU becomes the GroupNorm node followed by F.silu."""
    x, w3, g, b, x1, w1, b1 = _fake_cuda((1, 8, 4, 8, 8), (8, 8, 3, 3, 3), (8,), (8,), (2, 16, 64),
                                         (16, 1, 3), (16,), requires_grad=True)

    def f(x, w3, g, b, x1, w1, b1):
        y = amd_tuned_torch.group_norm_silu(F.conv3d(x, w3, None, 1, 1), 4, g, b, 1e-5)
        return y, F.conv1d(x1, w1, b1, padding=2, groups=16)

    (y, z), targets = _capture(f, x, w3, g, b, x1, w1, b1)
    names = [str(t) for t in targets]
    assert "amd_tuned_torch.conv3d_native" in names and "amd_tuned_torch.group_norm" in names
    assert "amd_tuned_torch.group_norm_silu" not in names
    assert z.shape == (2, 16, 66)


def test_custom_op_autograd_formulas_on_cpu():
    """The registered backward of the conv and GroupNorm ops (on CPU tensors their eager
    bodies take the stock paths) matches stock autograd; unrequested gradients stay None."""
    torch.manual_seed(0)
    x = torch.randn(2, 4, 5, 6, 6, dtype=torch.float64, requires_grad=True)
    w = torch.randn(6, 4, 3, 3, 3, dtype=torch.float64, requires_grad=True)
    b = torch.randn(6, dtype=torch.float64, requires_grad=True)
    y = ops.conv3d_native(x, w, b, [1, 1, 1], [1, 1, 1], [1, 1, 1])
    gy = torch.randn_like(y)
    got = torch.autograd.grad(y, (x, w, b), gy)
    ref = torch.autograd.grad(F.conv3d(x, w, b, 1, 1), (x, w, b), gy)
    for a, r in zip(got, ref):
        assert torch.allclose(a, r, atol=1e-10)
    y2 = ops.conv2d_native(x[:, :, 0], w[:, :, 0], None, [1, 1], [0, 0], [1, 1])
    (gx2,) = torch.autograd.grad(y2.sum(), (x,))
    (rx2,) = torch.autograd.grad(F.conv2d(x[:, :, 0], w[:, :, 0]).sum(), (x,))
    assert torch.allclose(gx2, rx2, atol=1e-10)

    xg = torch.randn(3, 8, 5, 5, dtype=torch.float64, requires_grad=True)
    gm = torch.randn(8, dtype=torch.float64, requires_grad=True)
    bt = torch.randn(8, dtype=torch.float64, requires_grad=True)
    out = ops.group_norm(xg, 4, gm, bt, 1e-5)
    go = torch.randn_like(out)
    got = torch.autograd.grad(out, (xg, gm, bt), go)
    ref = torch.autograd.grad(F.group_norm(xg, 4, gm, bt, 1e-5), (xg, gm, bt), go)
    for a, r in zip(got, ref):
        assert torch.allclose(a, r, atol=1e-9)
    # only the input needs a gradient: the parameter slots come back None
    xg2 = xg.detach().requires_grad_(True)
    (gx_only,) = torch.autograd.grad(ops.group_norm(xg2, 4, gm.detach(), bt.detach(), 1e-5).sum(), (xg2,))
    assert gx_only.shape == xg2.shape


def _real_vs_fake(op, *args):
    """(real outputs, fake outputs) of one custom op on the same arguments."""
    real = op(*args)
    with FakeTensorMode(allow_non_fake_inputs=True) as mode:
        fargs = [mode.from_tensor(a) if isinstance(a, torch.Tensor) else a for a in args]
        fake = op(*fargs)
    return real, fake


def test_group_norm_backward_op_outputs_match_its_fake():
    """The backward op's real outputs carry the dtypes and strides its fake promises, also when
    the eager body falls back to the torch-op backward (CPU here; on a GPU a shape the native
    kernels decline), which computes dgamma / dbeta in the parameter dtypes: a compiled graph
    built on the fake would otherwise read 2-byte gradients as float32."""
    torch.manual_seed(0)
    for dt, wdt, cl in ((torch.bfloat16, torch.bfloat16, False), (torch.float16, torch.float16, False),
                        (torch.bfloat16, torch.float32, False), (torch.bfloat16, torch.bfloat16, True)):
        x = torch.randn(2, 8, 14, 14).to(dt)
        if cl:
            x = x.contiguous(memory_format=torch.channels_last)
        dy = torch.randn(2, 8, 14, 14).to(dt).contiguous(memory_format=torch.channels_last if cl
                                                           else torch.contiguous_format)
        w = (1 + 0.1 * torch.randn(8)).to(wdt)
        real, fake = _real_vs_fake(ops.group_norm_backward, dy, x, 4, w, 1e-5, [True, True, True])
        for r, f in zip(real, fake):
            assert r.dtype == f.dtype and r.shape == f.shape and r.stride() == f.stride(), \
                (dt, wdt, cl, r.dtype, f.dtype, r.stride(), f.stride())
        # the conformed values are the fallback's own
        ref = torch.ops.aten.native_group_norm_backward(
            dy.float().contiguous(), x.float().contiguous(), *torch.ops.aten.native_group_norm(
                x.float().contiguous(), w.float(), None, 2, 8, 196, 4, 1e-5)[1:], w.float(), 2, 8, 196, 4,
            [True, True, True])
        assert torch.allclose(real[1], ref[1], rtol=2e-2, atol=2e-2)
        assert torch.allclose(real[2], ref[2], rtol=2e-2, atol=2e-2)


def test_conv_backward_op_outputs_match_its_fake():
    """Same check for the conv backward op (dx in the input's layout and dtype, dw in the
    weight's, db in the weight dtype)."""
    torch.manual_seed(0)
    x = torch.randn(1, 4, 6, 6).to(torch.bfloat16)
    w = (0.2 * torch.randn(6, 4, 3, 3)).to(torch.bfloat16)
    dy = torch.randn(1, 6, 6, 6).to(torch.bfloat16)
    real, fake = _real_vs_fake(ops.conv_backward, dy, x, w, True, [1, 1], [1, 1], [1, 1], 2,
                               [True, True, True])
    for r, f in zip(real, fake):
        assert r.dtype == f.dtype and r.shape == f.shape and r.stride() == f.stride()
