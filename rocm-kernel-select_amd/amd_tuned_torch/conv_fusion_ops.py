"""GroupNorm + SiLU fusion: `group_norm_silu`, `FusedGroupNormSiLUConv2d`,
`replace_conv_blocks` / `unfuse_conv_blocks`.

Interface and semantics of the reference's conv_fusion_ops (amd_tuned_torch/
conv_fusion_ops.py:169-451): SiLU(GroupNorm(x)) decided per shape by a kernel_select
contest keyed with the memory layout, stock = the captured ORIGINAL group_norm followed by
F.silu, forward-only (stock whenever a gradient is live).  The fused candidates are this
package's gfx950 GroupNorm variants with the SiLU applied in the normalisation epilogue
(one read + one write of the tensor), instead of the reference's Triton kernel.
AMD_TUNED_TORCH_CONV_FUSION=0 switches fusion off.
"""
from __future__ import annotations

import os
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _native
from . import kernel_select

_ENV = "AMD_TUNED_TORCH_CONV_FUSION"
_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def available() -> bool:
    """True when the fused path can run at all: native library loadable and a GPU visible."""
    return _native.available() and torch.cuda.is_available()


def enabled() -> bool:
    return available() and os.environ.get(_ENV, "1") != "0"


def _stock_group_norm_silu(x, num_groups, weight, bias, eps):
    """Unfused reference: the ORIGINAL F.group_norm (not the patched one), then SiLU."""
    try:
        from . import _dispatch
        gn = _dispatch._ORIGINALS.get((F, "group_norm"))
    except Exception:
        gn = None
    if gn is None:
        gn = torch.group_norm
    return F.silu(gn(x, num_groups, weight, bias, eps))


def _layout(x: torch.Tensor) -> str:
    if _native.is_channels_last(x):
        return "nhwc" if x.dim() == 4 else "ndhwc"
    return "nchw"


def _eligible(x, num_groups, weight, bias, layout_ok: bool = False) -> bool:
    """Native-eligible input: enabled, GPU, a supported dtype, contiguous (or, with
    layout_ok, any layout the caller handles), plain tensor types, no gradient needed."""
    if not (enabled() and isinstance(x, torch.Tensor) and x.is_cuda and x.dim() >= 3
            and x.dtype in _DTYPES and (layout_ok or x.is_contiguous())
            and type(x) in (torch.Tensor, nn.Parameter)):
        return False
    if not isinstance(num_groups, int) or num_groups <= 0 or x.shape[1] % num_groups != 0:
        return False
    for p in (weight, bias):
        if p is not None and (not p.is_cuda or p.dtype not in _DTYPES):
            return False
    if torch.is_grad_enabled() and (x.requires_grad or (weight is not None and weight.requires_grad)
                                    or (bias is not None and bias.requires_grad)):
        return False
    return True


def _grad_needed(x, weight, bias) -> bool:
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (x, weight, bias))


def _group_norm_silu_cl(x, num_groups, weight, bias, eps, stock):
    if not _eligible(x, num_groups, weight, bias, layout_ok=True):
        return stock()

    def native():
        try:
            return _native.group_norm_cl(x, num_groups, weight, bias, eps, silu=True)
        except _native.Unsupported:
            return None

    key = ("gn_silu", tuple(x.shape), str(x.dtype), num_groups, weight is not None,
           bias is not None, _layout(x))
    won = kernel_select.cached_key("group_norm_silu", key)
    if won == "stock":
        return stock()
    if won == "native.cl":
        out = native()
        if out is not None:
            return out
    out = kernel_select.pick_key("group_norm_silu", key, [("native.cl", native), ("stock", stock)])
    if out is not None:
        return out
    out = native()
    return out if out is not None else stock()


def group_norm_silu(x: torch.Tensor, num_groups: int, weight: Optional[torch.Tensor] = None,
                    bias: Optional[torch.Tensor] = None, eps: float = 1e-5) -> torch.Tensor:
    """SiLU(GroupNorm(x)) -- fused native kernel where it wins, stock where it does not.
    Channels-last input takes the NHWC / NDHWC kernel (`native.cl`) with the SiLU fused."""
    def stock():
        return _stock_group_norm_silu(x, num_groups, weight, bias, eps)

    if isinstance(x, torch.Tensor) and x.is_cuda and _grad_needed(x, weight, bias):
        # training: F.group_norm as installed (the native forward / backward when patched)
        return F.silu(F.group_norm(x, num_groups, weight, bias, eps))
    if isinstance(x, torch.Tensor) and x.is_cuda and _native.is_channels_last(x):
        return _group_norm_silu_cl(x, num_groups, weight, bias, eps, stock)
    if not _eligible(x, num_groups, weight, bias):
        return _stock_group_norm_silu(x, num_groups, weight, bias, eps)

    key = ("gn_silu", tuple(x.shape), str(x.dtype), num_groups, weight is not None,
           bias is not None, _layout(x))
    names = _native.variants(_native.OP_GROUP_NORM)
    won = kernel_select.cached_key("group_norm_silu", key)
    if won == "stock":
        return stock()
    if won is not None and won.startswith("native.") and won[7:] in names:
        try:
            return _native.group_norm(x, num_groups, weight, bias, eps, silu=True,
                                      variant=names.index(won[7:]))
        except _native.Unsupported:
            pass
    candidates = []
    for i, n in enumerate(names):
        def thunk(i=i):
            try:
                return _native.group_norm(x, num_groups, weight, bias, eps, silu=True, variant=i)
            except _native.Unsupported:
                return None
        candidates.append(("native." + n, thunk))
    candidates.append(("stock", stock))
    out = kernel_select.pick_key("group_norm_silu", key, candidates)
    if out is not None:
        return out
    for i in range(len(names)):  # kernel_select off: first variant that accepts the shape
        try:
            return _native.group_norm(x, num_groups, weight, bias, eps, silu=True, variant=i)
        except _native.Unsupported:
            continue
    return stock()


class FusedGroupNormSiLUConv2d(nn.Module):
    """Drop-in for nn.Sequential(GroupNorm, SiLU, Conv2d) holding the ORIGINAL submodules
    under the Sequential's indices "0" and "2", so parameters, optimizer state and
    state_dict keys survive (reference conv_fusion_ops.py:355-386)."""

    def __init__(self, norm: nn.GroupNorm, conv: nn.Conv2d):
        super().__init__()
        self.add_module("0", norm)
        self.add_module("2", conv)

    @property
    def norm(self) -> nn.GroupNorm:
        return getattr(self, "0")

    @property
    def conv(self) -> nn.Conv2d:
        return getattr(self, "2")

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        n = self.norm
        return self.conv(group_norm_silu(x, n.num_groups, n.weight, n.bias, n.eps))

    def extra_repr(self) -> str:
        return "fused=GroupNorm+SiLU"


class FusedConvGroupNormSiLU(nn.Module):
    """Drop-in for nn.Sequential(Conv2d | Conv3d, GroupNorm(affine), SiLU): the decoder-block
    order of a video VAE (Conv3d 256->256 k3 -> GroupNorm(32) -> SiLU).  The
    original submodules stay under the Sequential's indices "0" and "1", so parameters and
    state_dict keys survive.  The conv runs through F.conv2d / F.conv3d (the accelerated
    forward when patched), GroupNorm + SiLU through group_norm_silu: one fused pass over the
    conv output instead of a GroupNorm pass and a SiLU pass."""

    def __init__(self, conv: nn.Module, norm: nn.GroupNorm):
        super().__init__()
        self.add_module("0", conv)
        self.add_module("1", norm)

    @property
    def conv(self) -> nn.Module:
        return getattr(self, "0")

    @property
    def norm(self) -> nn.GroupNorm:
        return getattr(self, "1")

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        n = self.norm
        return group_norm_silu(self.conv(x), n.num_groups, n.weight, n.bias, n.eps)

    def extra_repr(self) -> str:
        return "fused=GroupNorm+SiLU after conv"


def _is_target(seq: nn.Module) -> bool:
    if not isinstance(seq, nn.Sequential) or len(seq) != 3:
        return False
    a, b, c = seq[0], seq[1], seq[2]
    return (isinstance(a, nn.GroupNorm) and a.affine and isinstance(b, nn.SiLU)
            and isinstance(c, nn.Conv2d))


def _is_vae_target(seq: nn.Module) -> bool:
    """nn.Sequential(Conv2d | Conv3d, GroupNorm(affine), SiLU)."""
    if not isinstance(seq, nn.Sequential) or len(seq) != 3:
        return False
    a, b, c = seq[0], seq[1], seq[2]
    return (isinstance(a, (nn.Conv2d, nn.Conv3d)) and isinstance(b, nn.GroupNorm) and b.affine
            and type(c) is nn.SiLU)


def replace_conv_blocks(model: nn.Module) -> int:
    """Replace every nn.Sequential(GroupNorm(affine), SiLU, Conv2d) under `model` (in place,
    recursively) with FusedGroupNormSiLUConv2d, and every nn.Sequential(Conv2d | Conv3d,
    GroupNorm(affine), SiLU) with FusedConvGroupNormSiLU; returns the count.  No-op (0) when
    fusion is not enabled.  Idempotent."""
    if not enabled():
        return 0
    n = 0
    for name, child in list(model.named_children()):
        if _is_target(child):
            setattr(model, name, FusedGroupNormSiLUConv2d(child[0], child[2]))
            n += 1
        elif _is_vae_target(child):
            setattr(model, name, FusedConvGroupNormSiLU(child[0], child[1]))
            n += 1
        else:
            n += replace_conv_blocks(child)
    return n


def unfuse_conv_blocks(model: nn.Module) -> int:
    """Undo replace_conv_blocks (same GroupNorm / conv objects, a fresh SiLU)."""
    n = 0
    for name, child in list(model.named_children()):
        if isinstance(child, FusedGroupNormSiLUConv2d):
            setattr(model, name, nn.Sequential(child.norm, nn.SiLU(), child.conv))
            n += 1
        elif isinstance(child, FusedConvGroupNormSiLU):
            setattr(model, name, nn.Sequential(child.conv, child.norm, nn.SiLU()))
            n += 1
        else:
            n += unfuse_conv_blocks(child)
    return n


def describe() -> str:
    if not _native.available():
        return "conv_fusion: unavailable -- native library not loadable"
    if not torch.cuda.is_available():
        return "conv_fusion: unavailable -- no GPU"
    if not enabled():
        return f"conv_fusion: disabled by {_ENV}=0"
    return ("conv_fusion: available -- GroupNorm+SiLU fused in the native GroupNorm epilogue, "
            "per-shape contest against stock via kernel_select")
