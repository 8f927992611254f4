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
from . import compile_ops
from . import kernel_select

_ENV = "AMD_TUNED_TORCH_CONV_FUSION"
_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def available() -> bool:
    """True when the fused path can run at all: native library loadable and a GPU visible."""
    return _native.available() and torch.cuda.is_available()


def enabled() -> bool:
    return available() and os.environ.get(_ENV, "1") != "0"


def _stock_group_norm_silu(x, num_groups, weight, bias, eps):
    """The selector's reference for the fused kernels: F.silu after the UNPATCHED GroupNorm
    (enable() replaces F.group_norm, so the one it captured is taken; aten's
    torch.group_norm when nothing was captured)."""
    from . import _dispatch  # imports this module, so resolved at call time
    stock_gn = _dispatch._STOCK_F.get("group_norm", torch.group_norm)
    return F.silu(stock_gn(x, num_groups, weight, bias, eps))


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


def _traced_group_norm_silu(x, num_groups, weight, bias, eps):
    """Under torch.compile: with a gradient live, the patched F.group_norm (its own graph node
    with the native backward) then F.silu; otherwise one forward-only graph node whose body
    runs this function's eager selection; stock outside the kernels' reach."""
    if _grad_needed(x, weight, bias):
        return F.silu(F.group_norm(x, num_groups, weight, bias, eps))
    ok = (os.environ.get(_ENV, "1") != "0" and compile_ops.native_loaded()
          and isinstance(x, torch.Tensor) and x.is_cuda and x.dim() >= 3 and x.dtype in _DTYPES
          and (x.is_contiguous() or _native.is_channels_last(x))
          and isinstance(num_groups, int) and num_groups > 0 and x.shape[1] % num_groups == 0
          and all(p is None or (p.is_cuda and p.dtype in _DTYPES) for p in (weight, bias)))
    if not ok:
        return _stock_group_norm_silu(x, num_groups, weight, bias, eps)
    return compile_ops.group_norm_silu(x, num_groups, weight, bias, eps)


def group_norm_silu(x: torch.Tensor, num_groups: int, weight: Optional[torch.Tensor] = None,
                    bias: Optional[torch.Tensor] = None, eps: float = 1e-5) -> torch.Tensor:
    """SiLU(GroupNorm(x)) -- fused native kernel where it wins, stock where it does not.
    Channels-last input takes the NHWC / NDHWC kernel (`native.cl`) with the SiLU fused."""
    def stock():
        return _stock_group_norm_silu(x, num_groups, weight, bias, eps)

    if compile_ops.is_compiling():
        return _traced_group_norm_silu(x, num_groups, weight, bias, eps)
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


# ---------------------------------------------------------------------------
# Conv epilogue fusion: the conv's MFMA epilogue adds a residual and / or writes the GroupNorm
# statistics of the values it stores, so a following GroupNorm (+ SiLU) is one apply pass over
# the conv output instead of a statistics pass and an apply pass.  Each entry point contests
# its fused form, per MFMA variant, against the stock sequence (the reference of the
# contest's verification), keyed on the whole block's shapes.
# ---------------------------------------------------------------------------
def _conv_geometry_ok(x, weight, bias, residual, stride, padding, dilation) -> bool:
    if not (isinstance(x, torch.Tensor) and isinstance(weight, torch.Tensor) and x.is_cuda
            and x.dim() in (4, 5) and weight.dim() == x.dim() and weight.shape[1] == x.shape[1]
            and x.dtype in _DTYPES and weight.dtype == x.dtype and not isinstance(padding, str)
            and x.is_contiguous() and weight.is_contiguous()
            and type(x) in (torch.Tensor, nn.Parameter) and _native.available()):
        return False
    for t in (bias, residual):
        if t is not None and (not t.is_cuda or t.dtype != x.dtype):
            return False
    return residual is None or residual.is_contiguous()


def _stock_conv_fn(nd: int):
    from . import _dispatch
    return _dispatch._STOCK_F["conv%dd" % nd]


def _mfma_variants(dtype) -> "list[tuple[int, str]]":
    names = _native.variants(_native.OP_CONV)
    prefix = "f32_" if dtype == torch.float32 else "h_"
    return [(i, n) for i, n in enumerate(names) if n.startswith(prefix)]


def _norm(v, nd):
    return (v,) * nd if isinstance(v, int) else tuple(v)


def conv_residual(input: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
                  residual: torch.Tensor, stride=1, padding=0, dilation=1) -> torch.Tensor:
    """conv2d / conv3d(input, weight, bias) + residual with the add in the conv's epilogue
    (groups = 1, zero padding): one write of the output instead of a write, a read of both
    and another write.  Falls back to the stock conv and an add (also when a gradient is
    needed)."""
    nd = input.dim() - 2 if isinstance(input, torch.Tensor) else 0
    stock_conv = _stock_conv_fn(nd) if nd in (2, 3) else None

    def stock():
        return stock_conv(input, weight, bias, stride, padding, dilation) + residual

    if (nd not in (2, 3) or _grad_needed(input, weight, bias) or _grad_needed(residual, None, None)
            or compile_ops.is_compiling()
            or not _conv_geometry_ok(input, weight, bias, residual, stride, padding, dilation)):
        return (stock_conv(input, weight, bias, stride, padding, dilation) if stock_conv is not None
                else F.conv3d(input, weight, bias, stride, padding, dilation)) + residual
    fn = _native.conv3d if nd == 3 else _native.conv2d

    def native(vi):
        def run():
            try:
                return fn(input, weight, bias, stride, padding, dilation, variant=vi, residual=residual)
            except _native.Unsupported:
                return None
        return run

    key = ("conv%dd" % nd, input.dtype, tuple(input.shape), tuple(weight.shape), _norm(stride, nd),
           _norm(padding, nd), _norm(dilation, nd), bias is not None)
    won = kernel_select.cached_key("conv_residual", key)
    if won == "stock":
        return stock()

    def unfused():  # the accelerated conv, then the add
        return (F.conv3d if nd == 3 else F.conv2d)(input, weight, bias, stride, padding, dilation) + residual
    if won == "native.unfused":
        return unfused()
    cands = [("native." + n, native(i)) for i, n in _mfma_variants(input.dtype)]
    cands.append(("native.unfused", unfused))
    if won is not None:
        for name, run in cands:
            if name == won:
                out = run()
                if out is not None:
                    return out
    out = kernel_select.pick_key("conv_residual", key, cands + [("stock", stock)])
    return out if out is not None else stock()


def conv_group_norm_silu(input: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], stride,
                         padding, dilation, num_groups: int, gamma: Optional[torch.Tensor],
                         beta: Optional[torch.Tensor], eps: float, silu: bool = True) -> torch.Tensor:
    """act(GroupNorm(conv(input, weight, bias))) for a groups-1, zero-padded conv2d / conv3d
    (act = SiLU or identity).  Candidates per MFMA variant: `native.<variant>` -- the conv's
    epilogue writes the GroupNorm statistics of its output, then one pass normalises it in
    place (two kernels) -- and `native.onepass.<variant>` -- one cooperative launch whose tiles
    stay in registers while the statistics are exchanged, so y is written once, normalised;
    plus the accelerated conv followed by the accelerated GroupNorm(+SiLU).  Falls back to the
    stock sequence (the reference of the contest) and, with a gradient live, to the patched
    functional path."""
    nd = input.dim() - 2 if isinstance(input, torch.Tensor) else 0

    def unfused_patched():
        conv = F.conv3d if nd == 3 else F.conv2d
        h = conv(input, weight, bias, stride, padding, dilation)
        return group_norm_silu(h, num_groups, gamma, beta, eps) if silu else F.group_norm(h, num_groups, gamma,
                                                                                          beta, eps)

    if (nd not in (2, 3) or compile_ops.is_compiling() or _grad_needed(input, weight, bias)
            or _grad_needed(gamma, beta, None) or not enabled()
            or not _conv_geometry_ok(input, weight, bias, None, stride, padding, dilation)
            or not isinstance(num_groups, int) or num_groups <= 0 or weight.shape[0] % num_groups
            or any(p is not None and (not p.is_cuda or p.dtype not in _DTYPES) for p in (gamma, beta))):
        return unfused_patched()
    stock_conv = _stock_conv_fn(nd)

    def stock():
        h = stock_conv(input, weight, bias, stride, padding, dilation)
        return _stock_group_norm_silu(h, num_groups, gamma, beta, eps) if silu else \
            _dispatch_stock_gn()(h, num_groups, gamma, beta, eps)

    fn = _native.conv_gn_stats

    def fused(vi):
        def run():
            try:
                y, rec, nrec = fn(input, weight, bias, stride, padding, dilation, nd, num_groups, variant=vi)
                return _native.group_norm_apply(y, num_groups, gamma, beta, eps, rec, nrec, silu=silu, out=y)
            except _native.Unsupported:
                return None
        return run

    def onepass(vi):
        def run():
            try:
                return _native.conv_group_norm(input, weight, bias, gamma, beta, stride, padding, dilation, nd,
                                               num_groups, eps, silu=silu, variant=vi)
            except _native.Unsupported:
                return None
        return run

    key = ("conv%dd" % nd, input.dtype, tuple(input.shape), tuple(weight.shape), _norm(stride, nd),
           _norm(padding, nd), _norm(dilation, nd), bias is not None, num_groups, silu,
           gamma is not None, beta is not None)
    won = kernel_select.cached_key("conv_group_norm", key)
    if won == "stock":
        return stock()
    if won == "native.unfused":
        return unfused_patched()
    # the fused form per MFMA variant, and the accelerated conv followed by the accelerated
    # GroupNorm(+SiLU) -- whichever is fastest for this block (the epilogue statistics cost
    # the conv a little; they pay only when they save more in the GroupNorm pass)
    cands = [("native." + n, fused(i)) for i, n in _mfma_variants(input.dtype)]
    if input.dtype in (torch.float16, torch.bfloat16):
        cands += [("native.onepass." + n, onepass(i)) for i, n in _mfma_variants(input.dtype)]
    cands.append(("native.unfused", unfused_patched))
    if won is not None:
        for name, run in cands:
            if name == won:
                out = run()
                if out is not None:
                    return out
    out = kernel_select.pick_key("conv_group_norm", key, cands + [("stock", stock)])
    return out if out is not None else stock()


def _dispatch_stock_gn():
    from . import _dispatch
    return _dispatch._STOCK_F.get("group_norm", torch.group_norm)


class _FusedBlock(nn.Module):
    """A fused replacement for a 3-module nn.Sequential that keeps the ORIGINAL conv and
    GroupNorm objects registered under their Sequential indices (the SiLU, which holds no
    state, is dropped): parameters, optimizer state and state_dict keys carry over unchanged
    (the reference's replace_conv_blocks contract, conv_fusion_ops.py:355-439)."""

    NORM_AT = CONV_AT = ""

    def __init__(self, norm: nn.GroupNorm, conv: nn.Module):
        super().__init__()
        for index, module in sorted(((self.NORM_AT, norm), (self.CONV_AT, conv))):
            self.add_module(index, module)

    @property
    def norm(self) -> nn.GroupNorm:
        return self._modules[self.NORM_AT]

    @property
    def conv(self) -> nn.Module:
        return self._modules[self.CONV_AT]

    def _gn_silu(self, h: torch.Tensor) -> torch.Tensor:
        n = self.norm
        return group_norm_silu(h, n.num_groups, n.weight, n.bias, n.eps)


class FusedGroupNormSiLUConv2d(_FusedBlock):
    """nn.Sequential(GroupNorm(affine), SiLU, Conv2d) -> GroupNorm+SiLU in one pass, then the
    conv.  Submodules "0" (GroupNorm) and "2" (Conv2d)."""

    NORM_AT, CONV_AT = "0", "2"

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.conv(self._gn_silu(x))

    def extra_repr(self) -> str:
        return "fused=GroupNorm+SiLU"


class FusedConvGroupNormSiLU(_FusedBlock):
    """nn.Sequential(Conv2d | Conv3d, GroupNorm(affine), SiLU): the decoder-block order of a
    video VAE (Conv3d 256->256 k3 -> GroupNorm(32) -> SiLU).  The conv runs
    through F.conv2d / F.conv3d (the accelerated forward when patched), GroupNorm + SiLU in
    one pass over its output.  Submodules "0" (conv) and "1" (GroupNorm)."""

    NORM_AT, CONV_AT = "1", "0"

    def __init__(self, conv: nn.Module, norm: nn.GroupNorm):
        super().__init__(norm, conv)

    @staticmethod
    def forward_parts(c: nn.Module, n: nn.GroupNorm, x: torch.Tensor) -> torch.Tensor:
        if (getattr(c, "padding_mode", "zeros") == "zeros" and getattr(c, "groups", 1) == 1
                and not isinstance(c.padding, str) and isinstance(x, torch.Tensor) and x.is_cuda):
            # GroupNorm statistics from the conv's epilogue, one apply pass (inference; with a
            # gradient live this is the patched conv followed by group_norm_silu)
            return conv_group_norm_silu(x, c.weight, c.bias, c.stride, c.padding, c.dilation, n.num_groups,
                                        n.weight, n.bias, n.eps)
        return group_norm_silu(c(x), n.num_groups, n.weight, n.bias, n.eps)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.forward_parts(self.conv, self.norm, x)

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
