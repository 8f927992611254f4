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
