"""The monkeypatch tier behind enable()/disable(): F.conv2d, F.conv3d, F.group_norm and
the nn.Sequential(GroupNorm, SiLU, Conv2d) fusion, plus eligibility checks, route
debugging and the TorchScript guard.

Behavioural restatement of the reference's conv/GroupNorm dispatch
(amd_tuned_torch/_dispatch.py:505-672 install/eligibility, 1617-2093 conv2d/conv3d,
2100-2370 group_norm, 2722-2738 Sequential fusion, 2913-3050 enable/disable, 3099-3155
TorchScript guard, 96-219 route debugging).  The candidate set is different by design:
instead of CK / FFT / aiter tiers, each contest is between this package's own gfx950
kernel variants ("native.<variant>") and stock, decided per shape by kernel_select.
"""
from __future__ import annotations

import atexit
import logging
import os
from typing import Any, Callable

import torch
import torch.nn.functional as F

from . import _native
from . import conv_fusion_ops
from . import kernel_select

# ---------------------------------------------------------------------------
# Route debugging (reference _dispatch.py:57-219): AMD_TUNED_TORCH_DISPATCH_DEBUG=1 or
# AMD_TUNED_TORCH_DISPATCH_DEBUG_FILE=<path>; every call site is `if _DEBUG: _debug(...)`.
# ---------------------------------------------------------------------------
_dbg_log = logging.getLogger("amd_tuned_torch.dispatch")
_DEBUG_ENV_SET = os.environ.get("AMD_TUNED_TORCH_DISPATCH_DEBUG", "0") not in ("0", "", "false", "False")
_DEBUG_FILE = os.environ.get("AMD_TUNED_TORCH_DISPATCH_DEBUG_FILE", "")
_DEBUG = _DEBUG_ENV_SET or bool(_DEBUG_FILE)

if _DEBUG:
    _dbg_log.setLevel(logging.DEBUG)
    _fmt = logging.Formatter("[amd_tuned_torch.dispatch] %(asctime)s %(levelname)s %(message)s")
    if _DEBUG_ENV_SET and not any(type(h) is logging.StreamHandler for h in _dbg_log.handlers):
        _h = logging.StreamHandler()
        _h.setFormatter(_fmt)
        _dbg_log.addHandler(_h)
    if _DEBUG_FILE and not any(isinstance(h, logging.FileHandler) for h in _dbg_log.handlers):
        _fh = logging.FileHandler(_DEBUG_FILE)
        _fh.setFormatter(_fmt)
        _dbg_log.addHandler(_fh)

_ROUTE_COUNTS: dict = {}


def _dbg_t(t: Any) -> str:
    if not isinstance(t, torch.Tensor):
        return repr(t)
    s = "%s%s" % (str(t.dtype).replace("torch.", ""), tuple(t.shape))
    if t.layout != torch.strided:
        s += ":" + str(t.layout).replace("torch.", "")
    if t.requires_grad:
        s += "+grad"
    if type(t) not in _PLAIN_TENSOR_TYPES:
        s += ":" + type(t).__name__
    return s


def _debug(op: str, route: str, why: str = "", **fields: Any) -> None:
    _ROUTE_COUNTS[(op, route)] = _ROUTE_COUNTS.get((op, route), 0) + 1
    if not _dbg_log.isEnabledFor(logging.DEBUG):
        return
    parts = ["%-10s -> %-16s" % (op, route)]
    if why:
        parts.append(why)
    for k, v in fields.items():
        parts.append("%s=%s" % (k, _dbg_t(v) if isinstance(v, torch.Tensor) else v))
    _dbg_log.debug("  ".join(parts))


def dispatch_debug_enabled() -> bool:
    return _DEBUG


def dispatch_debug_counts() -> dict:
    return dict(_ROUTE_COUNTS)


def dispatch_debug_reset() -> None:
    _ROUTE_COUNTS.clear()


def dispatch_debug_report() -> str:
    if not _ROUTE_COUNTS:
        return ("amd_tuned_torch dispatch: no routing decisions recorded"
                + ("" if _DEBUG else " (AMD_TUNED_TORCH_DISPATCH_DEBUG is not set)"))
    per_op: dict = {}
    for (op, route), n in _ROUTE_COUNTS.items():
        per_op.setdefault(op, {})[route] = n
    lines = ["amd_tuned_torch dispatch routes (%d decisions):" % sum(_ROUTE_COUNTS.values())]
    for op in sorted(per_op, key=lambda o: -sum(per_op[o].values())):
        tot = sum(per_op[op].values())
        lines.append("  %-12s %d" % (op, tot))
        for route in sorted(per_op[op], key=lambda r: -per_op[op][r]):
            n = per_op[op][route]
            lines.append("      %-18s %8d  %5.1f%%" % (route, n, 100.0 * n / tot))
    return "\n".join(lines)


def _dbg_atexit_report() -> None:
    if _ROUTE_COUNTS:
        _dbg_log.info("%s", dispatch_debug_report())


if _DEBUG:
    atexit.register(_dbg_atexit_report)

# Raw, unpatched handle on the native kernels (reference `ops = _C`).
ops = _native

_GROUPNORM_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
_CONV_NATIVE_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
_CONV3D_KIND = "conv3d"

_ORIGINALS: "dict[tuple[Any, str], Callable]" = {}
_ENABLED = False
_HAS_INFERENCE_MODE = hasattr(torch, "is_inference_mode_enabled")
_PLAIN_TENSOR_TYPES = (torch.Tensor, torch.nn.Parameter)


def _is_compiling() -> bool:
    try:
        return bool(torch.compiler.is_compiling())
    except AttributeError:
        try:
            return bool(torch._dynamo.is_compiling())
        except Exception:
            return False


def _grad_safe(*tensors: Any) -> bool:
    """True when no backward will run through this call (inference mode, no_grad, or no
    argument requires grad) -- reference _dispatch.py:528-553."""
    if _HAS_INFERENCE_MODE and torch.is_inference_mode_enabled():
        return True
    if not torch.is_grad_enabled():
        return True
    for t in tensors:
        if isinstance(t, torch.Tensor) and t.requires_grad:
            return False
    return True


def _is_plain_tensor(t: Any) -> bool:
    return type(t) in _PLAIN_TENSOR_TYPES


def _usable(*tensors: Any, dtypes: tuple = _CONV_NATIVE_DTYPES) -> bool:
    """Exact torch.Tensor/Parameter type (no subclasses), on the GPU, dtype in `dtypes`
    (reference _dispatch.py:643-659)."""
    for t in tensors:
        if not isinstance(t, torch.Tensor):
            continue
        if not _is_plain_tensor(t):
            return False
        if not t.is_cuda or t.dtype not in dtypes:
            return False
    return True


def _install(target: Any, name: str, wrapper: Callable) -> None:
    key = (target, name)
    if key not in _ORIGINALS:
        _ORIGINALS[key] = getattr(target, name)
    setattr(target, name, wrapper)


def _restore(target: Any, name: str) -> None:
    original = _ORIGINALS.pop((target, name), None)
    if original is not None:
        setattr(target, name, original)


def _triple(v):
    return (v, v, v) if isinstance(v, int) else tuple(v)


def _pair(v):
    return (v, v) if isinstance(v, int) else tuple(v)


# ---------------------------------------------------------------------------
# Native candidates
# ---------------------------------------------------------------------------
_NATIVE_PREFIX = "native."
_variant_cache: dict = {}


def _variants(op: int) -> "list[str]":
    v = _variant_cache.get(op)
    if v is None:
        v = _native.variants(op) if _native.available() else []
        _variant_cache[op] = v
    return v


def _native_thunk(fn: Callable, *args, **kwargs) -> Callable:
    """A candidate thunk: the native output, or None when the kernel declines the shape."""
    def thunk():
        try:
            return fn(*args, **kwargs)
        except _native.Unsupported:
            return None
    return thunk


def _conv_variant_names(dtype) -> "list[str]":
    """Conv variants worth contesting: the MFMA implicit-GEMM tiles, plus the direct
    kernel only when no implicit-GEMM variant exists in this build."""
    names = _variants(_native.OP_CONV)
    igemm = [n for n in names if n != "direct" and _conv_variant_dtype_ok(n, dtype)]
    return igemm if igemm else [n for n in names if n == "direct"]


def _conv_variant_dtype_ok(name: str, dtype) -> bool:
    """Variant names carry their operand class: "f32_*" fp32, "h_*" fp16/bf16."""
    if name.startswith("f32_"):
        return dtype == torch.float32
    if name.startswith("h"):
        return dtype in (torch.float16, torch.bfloat16)
    return True


def _conv_candidates(fn, input, weight, bias, stride, padding, dilation) -> list:
    out = []
    names = _variants(_native.OP_CONV)
    for name in _conv_variant_names(input.dtype):
        idx = names.index(name)
        out.append((_NATIVE_PREFIX + name,
                    _native_thunk(fn, input, weight, bias, stride, padding, dilation, variant=idx)))
    return out


def _run_named_native(name: str, fn: Callable, op: int, *args, **kwargs):
    """Run cached winner `name` ("native.<variant>"); None if it declines or is unknown."""
    try:
        idx = _variants(op).index(name[len(_NATIVE_PREFIX):])
    except ValueError:
        return None
    try:
        return fn(*args, variant=idx, **kwargs)
    except _native.Unsupported:
        return None


def _first_native(fn: Callable, op: int, names: "list[str]", *args, **kwargs):
    """Fixed-order fallback (kernel_select off): first variant that accepts the shape."""
    all_names = _variants(op)
    for name in names:
        try:
            return fn(*args, variant=all_names.index(name), **kwargs)
        except _native.Unsupported:
            continue
    return None


# ---------------------------------------------------------------------------
# conv2d / conv3d
# ---------------------------------------------------------------------------
def _is_pointwise_conv2d(weight, stride, padding, dilation) -> bool:
    """1x1 / stride 1 / pad 0 / dilation 1: a plain channel GEMM, left on stock
    (reference _dispatch.py:1351-1372)."""
    return (tuple(weight.shape[2:]) == (1, 1) and _pair(stride) == (1, 1)
            and _pair(padding) == (0, 0) and _pair(dilation) == (1, 1))


def _conv_accelerated_forward(nd: int, input, weight, bias, stride, padding, dilation, groups,
                              orig):
    op = "conv%dd" % nd
    kind = _CONV3D_KIND if nd == 3 else "conv2d"
    fn = _native.conv3d if nd == 3 else _native.conv2d
    if groups != 1:
        if _DEBUG:
            _debug(op, "stock", "grouped conv: no tier here supports groups != 1",
                   input=input, weight=weight, groups=groups)
        return orig(input, weight, bias, stride, padding, dilation, groups)
    eligible = (isinstance(input, torch.Tensor) and isinstance(weight, torch.Tensor)
                and not isinstance(padding, str)
                and input.dim() == nd + 2 and weight.dim() == nd + 2
                and (input.is_contiguous() or _channels_last(input))
                and (weight.is_contiguous() or _channels_last(weight))
                and _usable(input, weight, bias, dtypes=_CONV_NATIVE_DTYPES)
                and (bias is None or bias.dtype == input.dtype)
                and _native.available())
    if not eligible:
        if _DEBUG:
            _debug(op, "stock", "layout/dtype/device outside the native tier",
                   input=input, weight=weight)
        return orig(input, weight, bias, stride, padding, dilation, groups)
    if not (input.is_contiguous() and weight.is_contiguous()):
        # channels-last (NHWC / NDHWC) tensors: the MFMA kernels read NC(D)HW, so a native
        # candidate converts the input (and weight) and hands its output back in the input's
        # layout, as stock does; the contest times the conversions with the kernel, and the
        # winner cache keys on the memory format
        fn = _in_ncdhw(fn, _channels_last(input), nd)

    if kernel_select.enabled():
        won = kernel_select.cached(kind, input, weight, stride, padding, dilation)
        if won == "stock":
            if _DEBUG:
                _debug(op, "stock", "measured winner for this shape", input=input, weight=weight)
            return orig(input, weight, bias, stride, padding, dilation, groups)
        if won is not None and won.startswith(_NATIVE_PREFIX):
            out = _run_named_native(won, fn, _native.OP_CONV, input, weight, bias, stride,
                                    padding, dilation)
            if out is not None:
                if _DEBUG:
                    _debug(op, won, "cached winner", input=input, weight=weight)
                return out
            if _DEBUG:
                _debug(op, "declined", "cached winner %s declined" % won, input=input, weight=weight)
        candidates = _conv_candidates(fn, input, weight, bias, stride, padding, dilation)
        candidates.append(("stock", lambda: orig(input, weight, bias, stride, padding, dilation,
                                                 groups)))
        if _DEBUG:
            _debug(op, "contest", "first call for this shape", input=input, weight=weight,
                   candidates=",".join(n for n, _ in candidates))
        out = kernel_select.pick(kind, input, weight, stride, padding, dilation, candidates)
        if out is not None:
            if _DEBUG:
                _debug(op, kernel_select.cached(kind, input, weight, stride, padding, dilation)
                       or "unknown", "contest decided", input=input, weight=weight)
            return out

    # kernel_select off: first native variant that accepts the shape, then stock
    out = _first_native(fn, _native.OP_CONV, _conv_variant_names(input.dtype), input, weight,
                        bias, stride, padding, dilation)
    if out is not None:
        if _DEBUG:
            _debug(op, "native", "fixed order (kernel_select off)", input=input, weight=weight)
        return out
    if _DEBUG:
        _debug(op, "stock", "every native variant declined", input=input, weight=weight)
    return orig(input, weight, bias, stride, padding, dilation, groups)


def _to_ncdhw(t: torch.Tensor) -> torch.Tensor:
    """Contiguous form of a conv operand: channels-last tensors through the native
    transpose kernel, anything else through torch."""
    return _native.channels_last_to_contiguous(t) if _channels_last(t) else t.contiguous()


def _in_ncdhw(fn: Callable, cl_out: bool, nd: int) -> Callable:
    """`fn` on contiguous (NC(D)HW) copies of input and weight; the output converted to
    channels-last when `cl_out`.  The conversions run on the native transpose kernel."""

    def run(i, w, b, s, p, d, variant: int = -1):
        y = fn(_to_ncdhw(i), _to_ncdhw(w), b, s, p, d, variant=variant)
        return _native.contiguous_to_channels_last(y) if cl_out else y
    return run


def _dgrad_padding(weight, stride, padding, dilation, groups, nd):
    """Padding of the forward conv that computes the input gradient (k-1-p per dim), or None
    when that identity does not apply (stride or dilation != 1, groups != 1, string padding,
    p outside [0, k-1])."""
    tup = _triple if nd == 3 else _pair
    if groups != 1 or isinstance(padding, str):
        return None
    try:
        s, p, d = tup(stride), tup(padding), tup(dilation)
    except (TypeError, ValueError):
        return None
    if any(v != 1 for v in s) or any(v != 1 for v in d):
        return None
    ks = weight.shape[2:]
    if any(not (0 <= pi <= k - 1) for pi, k in zip(p, ks)):
        return None
    return [k - 1 - pi for pi, k in zip(p, ks)]


def _dgrad_via_forward(grad_output, weight, pad_t, nd, fwd):
    """dL/dx of a stride-1, dilation-1 conv: the forward conv of dy with the weights swapped
    in (Co, Ci) and flipped in space, padding k-1-p -- so the input gradient runs on the
    forward path (and its per-shape contest) instead of a separate dgrad."""
    wt = weight.transpose(0, 1).flip(list(range(2, 2 + nd))).contiguous()
    # a channels-last dy goes in as is: the forward path converts it with the native transpose
    dy = grad_output if _channels_last(grad_output) else grad_output.contiguous()
    return fwd(dy, wt, None, 1, pad_t, 1, 1)


def _wgrad_native(input, grad_output, weight, stride, padding, dilation, groups, nd):
    """Weight gradient through the native kernel for stride-1, dilation-1, groups-1 'same'
    convs with 3x3 (2D) or 3x3x3 / 1x3x3 (3D) kernels in 16-bit types; None otherwise (or when
    the kernel declines the shape)."""
    if groups != 1 or isinstance(padding, str) or weight.dtype not in (torch.float16, torch.bfloat16):
        return None
    tup = _triple if nd == 3 else _pair
    try:
        s, p, d = tup(stride), tup(padding), tup(dilation)
    except (TypeError, ValueError):
        return None
    if any(v != 1 for v in s) or any(v != 1 for v in d):
        return None
    k = tuple(weight.shape[2:])
    if nd == 3:
        if k not in ((3, 3, 3), (1, 3, 3)) or p != (k[0] // 2, 1, 1):
            return None
        kd, x5, g5 = k[0], input, grad_output
    else:
        if k != (3, 3) or p != (1, 1):
            return None
        kd, x5, g5 = 1, input.unsqueeze(2), grad_output.unsqueeze(2)
    if g5.dtype != x5.dtype or tuple(g5.shape[2:]) != tuple(x5.shape[2:]):
        return None
    try:
        dw = _native.conv_wgrad(_to_ncdhw(x5), _to_ncdhw(g5), kd)
    except _native.Unsupported:
        return None
    return dw.reshape(weight.shape).to(weight.dtype)


class _ConvFn(torch.autograd.Function):
    """Accelerated forward; the input gradient (stride 1, dilation 1, groups 1) through the
    same accelerated forward on dy with transposed, flipped weights; the weight gradient of
    'same' 3x3(x3) convs through the native wgrad kernel (and then the bias gradient as a
    reduction of dy); the rest through aten.convolution_backward -- the op autograd would
    have used unpatched (reference _Conv3dFn, _dispatch.py:2029-2075)."""

    @staticmethod
    def forward(ctx, input, weight, bias, stride, padding, dilation, groups, nd, fwd):
        ctx.save_for_backward(input, weight)
        ctx.bias_sizes = [bias.shape[0]] if bias is not None else None
        ctx.conf = (stride, padding, dilation, groups, nd)
        ctx.fwd = fwd
        return fwd(input, weight, bias, stride, padding, dilation, groups)

    @staticmethod
    def backward(ctx, grad_output):
        input, weight = ctx.saved_tensors
        stride, padding, dilation, groups, nd = ctx.conf
        needs = [bool(ctx.needs_input_grad[0]), bool(ctx.needs_input_grad[1]),
                 ctx.bias_sizes is not None and bool(ctx.needs_input_grad[2])]
        if not any(needs):
            return (None,) * 9
        gi = None
        if needs[0] and input.is_cuda:
            pad_t = _dgrad_padding(weight, stride, padding, dilation, groups, nd)
            if pad_t is not None:
                gi = _dgrad_via_forward(grad_output, weight.detach(), pad_t, nd, ctx.fwd)
                if tuple(gi.shape) != tuple(input.shape):
                    gi = None
                else:
                    needs[0] = False
        gw = gb = None
        if needs[1] and input.is_cuda:
            gw = _wgrad_native(input, grad_output, weight, stride, padding, dilation, groups, nd)
            if gw is not None:
                needs[1] = False
        if needs[2] and not needs[0] and not needs[1]:
            # every other gradient is native: the bias gradient is a reduction of dy
            gb = grad_output.sum(dim=[0] + list(range(2, 2 + nd)), dtype=torch.float32).to(weight.dtype)
            needs[2] = False
        if any(needs):
            tup = _triple if nd == 3 else _pair
            ai, aw, ab = torch.ops.aten.convolution_backward(
                grad_output.contiguous(), input, weight, ctx.bias_sizes, list(tup(stride)),
                list(tup(padding)), list(tup(dilation)), False, [0] * nd, groups, needs)
            gi = ai if gi is None else gi
            gw = aw if gw is None else gw
            gb = ab if gb is None else gb
        return gi, gw, gb, None, None, None, None, None, None


def _patched_conv2d(input, weight, bias=None, stride=1, padding=0, dilation=1, groups=1):
    orig = _ORIGINALS[(F, "conv2d")]
    if groups != 1:
        if _DEBUG:
            _debug("conv2d", "stock", "grouped conv: no tier here supports groups != 1",
                   input=input, weight=weight, groups=groups)
        return orig(input, weight, bias, stride, padding, dilation, groups)
    if (isinstance(weight, torch.Tensor) and weight.dim() == 4 and not isinstance(padding, str)
            and _is_pointwise_conv2d(weight, stride, padding, dilation)):
        if _DEBUG:
            _debug("conv2d", "stock", "1x1 pointwise conv", input=input, weight=weight)
        return orig(input, weight, bias, stride, padding, dilation, groups)

    def fwd(i, w, b, s, p, d, g):
        return _conv_accelerated_forward(2, i, w, b, s, p, d, g, orig)

    if _grad_safe(input, weight, bias):
        return fwd(input, weight, bias, stride, padding, dilation, groups)
    if _DEBUG:
        _debug("conv2d", "autograd", "gradient needed: accelerated fwd + stock backward",
               input=input, weight=weight)
    return _ConvFn.apply(input, weight, bias, stride, padding, dilation, groups, 2, fwd)


def _patched_conv3d(input, weight, bias=None, stride=1, padding=0, dilation=1, groups=1):
    orig = _ORIGINALS[(F, "conv3d")]

    def fwd(i, w, b, s, p, d, g):
        return _conv_accelerated_forward(3, i, w, b, s, p, d, g, orig)

    if _grad_safe(input, weight, bias):
        return fwd(input, weight, bias, stride, padding, dilation, groups)
    if groups != 1:
        if _DEBUG:
            _debug("conv3d", "stock", "grouped conv: no tier here supports groups != 1",
                   input=input, weight=weight, groups=groups)
        return orig(input, weight, bias, stride, padding, dilation, groups)
    if _DEBUG:
        _debug("conv3d", "autograd", "gradient needed: accelerated fwd + stock backward",
               input=input, weight=weight)
    return _ConvFn.apply(input, weight, bias, stride, padding, dilation, groups, 3, fwd)


# ---------------------------------------------------------------------------
# group_norm
# ---------------------------------------------------------------------------
def group_norm_variant_order(input: torch.Tensor) -> "list[str]":
    """Native GroupNorm variants in fixed-order preference (used when kernel_select is
    off): register-resident kernels first, the two-pass kernel last."""
    names = _variants(_native.OP_GROUP_NORM)
    res = [n for n in names if n.startswith("res_")]
    return res + [n for n in names if not n.startswith("res_")]


def _group_norm_candidates(input, num_groups, weight, bias, eps, silu: bool = False) -> list:
    names = _variants(_native.OP_GROUP_NORM)
    return [(_NATIVE_PREFIX + n,
             _native_thunk(_native.group_norm, input, num_groups, weight, bias, eps, silu=silu,
                           variant=i))
            for i, n in enumerate(names)]


def _group_norm_native(input, num_groups, weight, bias, eps, name=None):
    """Native GroupNorm: the named variant, or the first one that accepts the shape.
    Under Dynamo tracing the torch.library op is used instead (graph-break free)."""
    if _is_compiling():
        from . import compile_ops
        return compile_ops.group_norm(input, num_groups, weight, bias, eps)
    if name is not None:
        return _run_named_native(name, _native.group_norm, _native.OP_GROUP_NORM, input,
                                 num_groups, weight, bias, eps)
    return _first_native(_native.group_norm, _native.OP_GROUP_NORM,
                         group_norm_variant_order(input), input, num_groups, weight, bias, eps)


def _channels_last(x: torch.Tensor) -> bool:
    if x.dim() == 4:
        return x.is_contiguous(memory_format=torch.channels_last) and not x.is_contiguous()
    if x.dim() == 5:
        return x.is_contiguous(memory_format=torch.channels_last_3d) and not x.is_contiguous()
    return False


def _group_norm_channels_last(input, num_groups, weight, bias, eps, orig):
    """Channels-last input: one native candidate (`native.cl`, the NHWC / NDHWC kernel)
    against stock, keyed with the memory format like every GroupNorm contest (the
    reference contests CK there, _dispatch.py:2140-2200)."""
    if not (_usable(input, dtypes=_GROUPNORM_DTYPES) and _usable(weight, bias, dtypes=_GROUPNORM_DTYPES)
            and isinstance(num_groups, int) and num_groups > 0 and input.shape[1] % num_groups == 0
            and _native.available() and not _is_compiling()):
        if _DEBUG:
            _debug("group_norm", "stock", "channels-last outside this tier", input=input)
        return orig(input, num_groups, weight, bias, eps)
    native = _native_thunk(_native.group_norm_cl, input, num_groups, weight, bias, eps)
    if kernel_select.enabled():
        key = (input.dtype, tuple(input.shape), int(num_groups), True)
        won = kernel_select.cached_key("group_norm", key)
        if won == _NATIVE_PREFIX + "cl":
            out = native()
            if out is not None:
                return out
        elif won == "stock":
            return orig(input, num_groups, weight, bias, eps)
        out = kernel_select.pick_key("group_norm", key, [
            (_NATIVE_PREFIX + "cl", native),
            ("stock", lambda: orig(input, num_groups, weight, bias, eps))])
        if out is not None:
            return out
    out = native()
    return out if out is not None else orig(input, num_groups, weight, bias, eps)


def _group_norm_accelerated_forward(input, num_groups, weight, bias, eps):
    orig = _ORIGINALS[(F, "group_norm")]
    if isinstance(input, torch.Tensor) and _channels_last(input):
        return _group_norm_channels_last(input, num_groups, weight, bias, eps, orig)
    if not (isinstance(input, torch.Tensor) and input.dim() >= 2 and input.is_contiguous()
            and _usable(input, dtypes=_GROUPNORM_DTYPES)
            and _usable(weight, bias, dtypes=_GROUPNORM_DTYPES)
            and isinstance(num_groups, int) and num_groups > 0
            and input.shape[1] % num_groups == 0 and _native.available()):
        if _DEBUG:
            _debug("group_norm", "stock", "layout/dtype outside this tier", input=input)
        return orig(input, num_groups, weight, bias, eps)
    channels_last = _channels_last(input)
    if kernel_select.enabled():
        key = (input.dtype, tuple(input.shape), int(num_groups), channels_last)
        won = kernel_select.cached_key("group_norm", key)
        if won == "stock":
            if _DEBUG:
                _debug("group_norm", "stock", "measured winner for this shape", key=key)
            return orig(input, num_groups, weight, bias, eps)
        if won is not None and won.startswith(_NATIVE_PREFIX):
            out = _group_norm_native(input, num_groups, weight, bias, eps, name=won)
            if out is not None:
                if _DEBUG:
                    _debug("group_norm", won, "cached winner", key=key)
                return out
        candidates = _group_norm_candidates(input, num_groups, weight, bias, eps)
        candidates.append(("stock", lambda: orig(input, num_groups, weight, bias, eps)))
        if _DEBUG:
            _debug("group_norm", "contest", "first call for this shape", key=key,
                   candidates=",".join(n for n, _ in candidates))
        out = kernel_select.pick_key("group_norm", key, candidates)
        if out is not None:
            return out
    out = _group_norm_native(input, num_groups, weight, bias, eps)
    if out is not None:
        if _DEBUG:
            _debug("group_norm", "native", "fixed order (kernel_select off)", input=input)
        return out
    if _DEBUG:
        _debug("group_norm", "stock", "every native variant declined", input=input)
    return orig(input, num_groups, weight, bias, eps)


def _group_norm_backward(grad_output, input, num_groups, weight, eps, needs, bias_dtype=None):
    """GroupNorm's derivative in torch ops over an (N, G, M, S) view, reductions promoted to
    fp32 for 16-bit inputs (reference _dispatch.py:2212-2302):
        dx = rstd * (w*dy - mean(w*dy) - x_hat * mean(w*dy * x_hat)),
        dgamma = sum(dy * x_hat), dbeta = sum(dy)."""
    N, C = input.shape[0], input.shape[1]
    G = num_groups
    M = C // G
    dt = input.dtype
    acc = torch.float32 if dt in (torch.float16, torch.bfloat16) else dt
    x = input.reshape(N, G, M, -1)
    dy = grad_output.reshape(N, G, M, -1)
    need_x, need_w, need_b = needs
    gx = gw = gb = None
    if need_b:
        gb = dy.sum(dim=(0, 3), dtype=acc).reshape(C).to(bias_dtype if bias_dtype is not None else dt)
    if not (need_x or need_w):
        return gx, gw, gb
    mean = x.mean(dim=(2, 3), keepdim=True, dtype=acc)
    xc = x - mean.to(dt)
    var = xc.square().mean(dim=(2, 3), keepdim=True, dtype=acc)
    rstd = (var + eps).rsqrt().to(dt)
    x_hat = xc * rstd
    if need_w and weight is not None:
        gw = (dy * x_hat).sum(dim=(0, 3), dtype=acc).reshape(C).to(weight.dtype)
    if need_x:
        wdy = dy if weight is None else dy * weight.reshape(1, G, M, 1)
        c1 = wdy.mean(dim=(2, 3), keepdim=True, dtype=acc).to(dt)
        c2 = (wdy * x_hat).mean(dim=(2, 3), keepdim=True, dtype=acc).to(dt)
        gx = ((wdy - c1 - x_hat * c2) * rstd).reshape(input.shape)
        if _channels_last(input):
            gx = gx.contiguous(memory_format=torch.channels_last if input.dim() == 4
                               else torch.channels_last_3d)
    return gx, gw, gb


class _GroupNormFn(torch.autograd.Function):
    """Accelerated forward; native backward kernels (atk_group_norm_bwd) for contiguous GPU
    inputs, the textbook torch-op backward otherwise (reference _GroupNormFn, 2305-2359)."""

    @staticmethod
    def forward(ctx, input, weight, bias, num_groups, eps):
        ctx.save_for_backward(input, weight)
        ctx.num_groups, ctx.eps = num_groups, eps
        ctx.has_bias = bias is not None
        ctx.bias_dtype = bias.dtype if bias is not None else None
        return _group_norm_accelerated_forward(input, num_groups, weight, bias, eps)

    @staticmethod
    def backward(ctx, grad_output):
        input, weight = ctx.saved_tensors
        needs = (ctx.needs_input_grad[0], weight is not None and ctx.needs_input_grad[1],
                 ctx.has_bias and ctx.needs_input_grad[2])
        cl = _channels_last(input)
        if input.is_cuda and (input.is_contiguous() or cl) and _native.available():
            try:
                # channels-last x and dy go to NC[S] through the native transpose, and dx
                # comes back in the input's layout
                x = _native.channels_last_to_contiguous(input.detach()) if cl else input.detach()
                gx, gw, gb = _native.group_norm_backward(_to_ncdhw(grad_output), x, ctx.num_groups,
                                                         None if weight is None else weight.detach(),
                                                         ctx.eps, needs)
                if cl and gx is not None:
                    gx = _native.contiguous_to_channels_last(gx)
                gw = None if gw is None else gw.to(weight.dtype)
                gb = None if gb is None else gb.to(ctx.bias_dtype if ctx.bias_dtype is not None
                                                   else input.dtype)
                return gx, gw, gb, None, None
            except _native.Unsupported:
                pass
        return _group_norm_backward(grad_output.contiguous(), input, ctx.num_groups, weight,
                                    ctx.eps, needs, bias_dtype=ctx.bias_dtype) + (None, None)


def _patched_group_norm(input, num_groups, weight=None, bias=None, eps=1e-5):
    if _grad_safe(input, weight, bias):
        return _group_norm_accelerated_forward(input, num_groups, weight, bias, eps)
    if _DEBUG:
        _debug("group_norm", "autograd", "gradient needed: accelerated fwd + real backward",
               input=input)
    return _GroupNormFn.apply(input, weight, bias, num_groups, eps)


# ---------------------------------------------------------------------------
# nn.Sequential(GroupNorm(affine), SiLU, Conv2d) auto-fusion (reference 2722-2738), and the
# conv-first order nn.Sequential(Conv2d | Conv3d, GroupNorm(affine), SiLU)
# ---------------------------------------------------------------------------
_SEQ_FORWARD_ORIG = None


def _patched_sequential_forward(self, input):
    mods = self._modules
    if len(mods) == 3:
        norm, act, conv = mods.values()
        if (type(act) is torch.nn.SiLU and isinstance(norm, torch.nn.GroupNorm) and norm.affine
                and isinstance(conv, torch.nn.Conv2d)):
            if _DEBUG:
                _debug("sequential", "conv_fusion", "GroupNorm+SiLU fused", input=input)
            h = conv_fusion_ops.group_norm_silu(input, norm.num_groups, norm.weight, norm.bias,
                                                norm.eps)
            return conv(h)
        # the decoder-block order of a video VAE: Conv2d | Conv3d, GroupNorm(affine), SiLU
        conv, norm, act = mods.values()
        if (type(act) is torch.nn.SiLU and isinstance(norm, torch.nn.GroupNorm) and norm.affine
                and isinstance(conv, (torch.nn.Conv2d, torch.nn.Conv3d))):
            if _DEBUG:
                _debug("sequential", "conv_fusion", "conv then GroupNorm+SiLU fused", input=input)
            return conv_fusion_ops.group_norm_silu(conv(input), norm.num_groups, norm.weight, norm.bias,
                                                   norm.eps)
    return _SEQ_FORWARD_ORIG(self, input)


# ---------------------------------------------------------------------------
# enable / disable
# ---------------------------------------------------------------------------
def enable() -> None:
    """Patch torch.nn.functional so eligible calls route through amd_tuned_torch."""
    global _ENABLED, _SEQ_FORWARD_ORIG
    if _ENABLED:
        if _DEBUG:
            _debug("enable", "noop", "already enabled")
        return
    if _DEBUG:
        _debug("enable", "backends", "", native=_native.available(),
               kernel_select=kernel_select.enabled(), conv_fusion=conv_fusion_ops.enabled())
    _install(F, "group_norm", _patched_group_norm)
    _install(F, "conv2d", _patched_conv2d)
    if conv_fusion_ops.enabled():
        _install(torch.nn.Sequential, "forward", _patched_sequential_forward)
        _SEQ_FORWARD_ORIG = _ORIGINALS[(torch.nn.Sequential, "forward")]
    if hasattr(F, "conv3d"):
        _install(F, "conv3d", _patched_conv3d)
    _ENABLED = True
    if _DEBUG:
        _debug("enable", "installed", "", patched=",".join(sorted(n for _, n in _ORIGINALS)))


def disable() -> None:
    """Restore every function enable() patched."""
    global _ENABLED
    if _DEBUG:
        _debug("disable", "restored", "", patched=",".join(sorted(n for _, n in _ORIGINALS)))
    for target, name in list(_ORIGINALS.keys()):
        _restore(target, name)
    _ENABLED = False


def is_enabled() -> bool:
    return _ENABLED


# ---------------------------------------------------------------------------
# TorchScript guard (reference 3099-3155): script/trace compile against stock ops, since a
# scripted or traced graph cannot call these Python wrappers.  Installed at import time.
# ---------------------------------------------------------------------------
_ORIG_JIT_SCRIPT = torch.jit.script
_ORIG_JIT_TRACE = torch.jit.trace


def _script_with_stock_ops(obj, *args, **kwargs):
    # one extra Python frame between the caller and torch.jit.script: class scripting
    # resolves names _frames_up frames above, so compensate
    if len(args) >= 2:
        args = args[:1] + (args[1] + 1,) + args[2:]
    else:
        kwargs["_frames_up"] = kwargs.get("_frames_up", 0) + 1
    if not _ENABLED:
        return _ORIG_JIT_SCRIPT(obj, *args, **kwargs)
    disable()
    try:
        return _ORIG_JIT_SCRIPT(obj, *args, **kwargs)
    finally:
        enable()


def _trace_with_stock_ops(*args, **kwargs):
    if not _ENABLED:
        return _ORIG_JIT_TRACE(*args, **kwargs)
    disable()
    try:
        return _ORIG_JIT_TRACE(*args, **kwargs)
    finally:
        enable()


_script_with_stock_ops.__doc__ = _ORIG_JIT_SCRIPT.__doc__
_trace_with_stock_ops.__doc__ = _ORIG_JIT_TRACE.__doc__
torch.jit.script = _script_with_stock_ops
torch.jit.trace = _trace_with_stock_ops

__all__ = [
    "ops", "_dbg_log", "_DEBUG", "_DEBUG_ENV_SET", "_DEBUG_FILE", "_ROUTE_COUNTS", "_debug",
    "_dbg_t", "dispatch_debug_enabled", "dispatch_debug_counts", "dispatch_debug_reset",
    "dispatch_debug_report", "_GROUPNORM_DTYPES", "_CONV_NATIVE_DTYPES", "_CONV3D_KIND",
    "_ORIGINALS", "_ENABLED", "_HAS_INFERENCE_MODE", "_PLAIN_TENSOR_TYPES", "_is_compiling",
    "_grad_safe", "_is_plain_tensor", "_usable", "_install", "_restore", "_triple", "_pair",
    "_is_pointwise_conv2d", "_conv_accelerated_forward", "_ConvFn", "_patched_conv2d",
    "_patched_conv3d", "_group_norm_native", "_group_norm_accelerated_forward",
    "_group_norm_backward", "_GroupNormFn", "_dgrad_padding", "_dgrad_via_forward",
    "_patched_group_norm", "_patched_sequential_forward",
    "enable", "disable", "is_enabled", "_ORIG_JIT_SCRIPT", "_ORIG_JIT_TRACE",
    "_script_with_stock_ops", "_trace_with_stock_ops",
]
