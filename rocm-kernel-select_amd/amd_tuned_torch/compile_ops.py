"""torch.library custom ops over the native kernels, so torch.compile places them as opaque
graph nodes instead of breaking the graph at a ctypes call.

Names, schemas and fake (meta) implementations follow the reference's compile_ops
(amd_tuned_torch/compile_ops.py:168-235,369-415): `amd_tuned_torch::group_norm`,
`amd_tuned_torch::conv2d_native`, `amd_tuned_torch::conv3d_native`; the conv fakes reuse
aten's own conv meta kernels for the output size.  Registered for all device types;
eligibility is checked by the dispatch layer before these are called.  Forward only.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _native


def _already_registered(name: str) -> bool:
    return hasattr(torch.ops, "amd_tuned_torch") and hasattr(torch.ops.amd_tuned_torch, name)


def _triple(v):
    return (v, v, v) if isinstance(v, int) else tuple(v)


def _pair(v):
    return (v, v) if isinstance(v, int) else tuple(v)


if hasattr(torch.library, "custom_op") and not _already_registered("group_norm"):

    @torch.library.custom_op("amd_tuned_torch::group_norm", mutates_args=())
    def _group_norm_op(input_: torch.Tensor, num_groups: int, weight: Optional[torch.Tensor],
                       bias: Optional[torch.Tensor], eps: float) -> torch.Tensor:
        from ._dispatch import _first_native, group_norm_variant_order
        out = _first_native(_native.group_norm, _native.OP_GROUP_NORM,
                            group_norm_variant_order(input_), input_, num_groups, weight, bias, eps)
        if out is None:
            raise RuntimeError("amd_tuned_torch::group_norm: no native variant accepts this shape")
        return out

    @_group_norm_op.register_fake
    def _group_norm_fake(input_, num_groups, weight, bias, eps):
        return input_.new_empty(input_.shape)

    @torch.library.custom_op("amd_tuned_torch::conv2d_native", mutates_args=())
    def _conv2d_native_op(input_: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
                          stride: list[int], padding: list[int], dilation: list[int]) -> torch.Tensor:
        return _native.conv2d(input_, weight, bias, stride, padding, dilation)

    @_conv2d_native_op.register_fake
    def _conv2d_native_fake(input_, weight, bias, stride, padding, dilation):
        return torch.ops.aten.conv2d.default(input_, weight, bias, stride, padding, dilation, 1)

    @torch.library.custom_op("amd_tuned_torch::conv3d_native", mutates_args=())
    def _conv3d_native_op(input_: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
                          stride: list[int], padding: list[int], dilation: list[int]) -> torch.Tensor:
        return _native.conv3d(input_, weight, bias, stride, padding, dilation)

    @_conv3d_native_op.register_fake
    def _conv3d_native_fake(input_, weight, bias, stride, padding, dilation):
        return torch.ops.aten.conv3d.default(input_, weight, bias, stride, padding, dilation, 1)

    _group_norm_impl = torch.ops.amd_tuned_torch.group_norm
    _conv2d_native_impl = torch.ops.amd_tuned_torch.conv2d_native
    _conv3d_native_impl = torch.ops.amd_tuned_torch.conv3d_native
elif _already_registered("group_norm"):
    _group_norm_impl = torch.ops.amd_tuned_torch.group_norm
    _conv2d_native_impl = torch.ops.amd_tuned_torch.conv2d_native
    _conv3d_native_impl = torch.ops.amd_tuned_torch.conv3d_native
else:  # torch without torch.library.custom_op: same numerics, no graph node
    def _group_norm_impl(input_, num_groups, weight, bias, eps):
        return _native.group_norm(input_, num_groups, weight, bias, eps)

    def _conv2d_native_impl(input_, weight, bias, stride, padding, dilation):
        return _native.conv2d(input_, weight, bias, stride, padding, dilation)

    def _conv3d_native_impl(input_, weight, bias, stride, padding, dilation):
        return _native.conv3d(input_, weight, bias, stride, padding, dilation)


def group_norm(input_: torch.Tensor, num_groups: int, weight: Optional[torch.Tensor] = None,
               bias: Optional[torch.Tensor] = None, eps: float = 1e-5) -> torch.Tensor:
    return _group_norm_impl(input_, num_groups, weight, bias, eps)


def conv2d_native(input_, weight, bias=None, stride=1, padding=0, dilation=1) -> torch.Tensor:
    """gfx950 implicit-GEMM conv2d (groups = 1; fp16/bf16/fp32)."""
    return _conv2d_native_impl(input_, weight, bias, list(_pair(stride)), list(_pair(padding)),
                               list(_pair(dilation)))


def conv3d_native(input_, weight, bias=None, stride=1, padding=0, dilation=1) -> torch.Tensor:
    """gfx950 implicit-GEMM conv3d (groups = 1; fp16/bf16/fp32)."""
    return _conv3d_native_impl(input_, weight, bias, list(_triple(stride)),
                               list(_triple(padding)), list(_triple(dilation)))
