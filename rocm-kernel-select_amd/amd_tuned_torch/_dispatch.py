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
import collections
import contextlib
import functools
import inspect
import logging
import os
from typing import Any, Callable

import torch
import torch.nn.functional as F

from . import _native
from . import compile_ops
from . import conv_fusion_ops
from . import kernel_select


# ---------------------------------------------------------------------------
# Route debugging (the reference's AMD_TUNED_TORCH_DISPATCH_DEBUG / _DEBUG_FILE switches and
# dispatch_debug_* API, _dispatch.py:57-219).  Every call site is `if _DEBUG: _debug(...)`,
# so with the switches unset a decision costs one global read.
# ---------------------------------------------------------------------------
class _RouteLog:
    """Counts (op, route) decisions and, when the logger is at DEBUG, writes one line each."""

    def __init__(self, logger: logging.Logger):
        self.logger = logger
        self.counts: "collections.Counter[tuple[str, str]]" = collections.Counter()

    @staticmethod
    def describe(v: Any) -> str:
        """dtype(shape) of a tensor, plus layout / grad / subclass marks when they apply."""
        if not isinstance(v, torch.Tensor):
            return repr(v)
        marks = []
        if v.layout != torch.strided:
            marks.append(str(v.layout).rsplit(".", 1)[-1])
        if v.requires_grad:
            marks.append("grad")
        if type(v) not in _PLAIN_TENSOR_TYPES:
            marks.append(type(v).__name__)
        base = "%s%s" % (str(v.dtype).rsplit(".", 1)[-1], tuple(v.shape))
        return base + "".join("[%s]" % m for m in marks)

    def record(self, op: str, route: str, why: str, fields: dict) -> None:
        self.counts[(op, route)] += 1
        if self.logger.isEnabledFor(logging.DEBUG):
            text = "%s -> %s" % (op, route)
            if why:
                text += " (%s)" % why
            if fields:
                text += " " + " ".join("%s=%s" % (k, self.describe(v)) for k, v in fields.items())
            self.logger.debug(text)

    def report(self) -> str:
        if not self.counts:
            return ("amd_tuned_torch dispatch: no routing decisions recorded"
                    + ("" if _DEBUG else " (AMD_TUNED_TORCH_DISPATCH_DEBUG is not set)"))
        by_op: "dict[str, collections.Counter]" = collections.defaultdict(collections.Counter)
        for (op, route), n in self.counts.items():
            by_op[op][route] += n
        out = ["amd_tuned_torch dispatch routes (%d decisions):" % sum(self.counts.values())]
        for op, routes in sorted(by_op.items(), key=lambda kv: -sum(kv[1].values())):
            total = sum(routes.values())
            out.append("  %-12s %d" % (op, total))
            out.extend("      %-18s %8d  %5.1f%%" % (r, n, 100.0 * n / total)
                       for r, n in routes.most_common())
        return "\n".join(out)


def _debug_switches() -> "tuple[bool, str]":
    flag = os.environ.get("AMD_TUNED_TORCH_DISPATCH_DEBUG", "0").strip() not in ("", "0", "false", "False")
    return flag, os.environ.get("AMD_TUNED_TORCH_DISPATCH_DEBUG_FILE", "")


_dbg_log = logging.getLogger("amd_tuned_torch.dispatch")
_DEBUG_ENV_SET, _DEBUG_FILE = _debug_switches()
_DEBUG = _DEBUG_ENV_SET or bool(_DEBUG_FILE)
_ROUTES = _RouteLog(_dbg_log)
_ROUTE_COUNTS = _ROUTES.counts

if _DEBUG:
    _dbg_log.setLevel(logging.DEBUG)
    _line_format = logging.Formatter("[amd_tuned_torch.dispatch] %(asctime)s %(levelname)s %(message)s")
    _sinks = []
    if _DEBUG_ENV_SET and not any(type(h) is logging.StreamHandler for h in _dbg_log.handlers):
        _sinks.append(logging.StreamHandler())
    if _DEBUG_FILE and not any(isinstance(h, logging.FileHandler) for h in _dbg_log.handlers):
        _sinks.append(logging.FileHandler(_DEBUG_FILE))
    for _sink in _sinks:
        _sink.setFormatter(_line_format)
        _dbg_log.addHandler(_sink)
    atexit.register(lambda: _ROUTES.counts and _dbg_log.info("%s", _ROUTES.report()))


def _dbg_t(t: Any) -> str:
    return _RouteLog.describe(t)


def _debug(op: str, route: str, why: str = "", **fields: Any) -> None:
    _ROUTES.record(op, route, why, fields)


def dispatch_debug_enabled() -> bool:
    return _DEBUG


def dispatch_debug_counts() -> dict:
    return dict(_ROUTES.counts)


def dispatch_debug_reset() -> None:
    _ROUTES.counts.clear()


def dispatch_debug_report() -> str:
    return _ROUTES.report()


# Raw, unpatched handle on the native kernels (reference `ops = _C`).
ops = _native

_GROUPNORM_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
_CONV_NATIVE_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
_CONV3D_KIND = "conv3d"

_ORIGINALS: "dict[tuple[Any, str], Callable]" = {}
# The stock torch.nn.functional entry points by name, as _install found them: the patched
# functions read them from here (a string-keyed dict, which torch.compile can trace; a
# module-keyed one it cannot).
_STOCK_F: "dict[str, Callable]" = {n: getattr(F, n) for n in ("conv2d", "conv3d", "group_norm") if hasattr(F, n)}
_ENABLED = False
_HAS_INFERENCE_MODE = hasattr(torch, "is_inference_mode_enabled")
_PLAIN_TENSOR_TYPES = (torch.Tensor, torch.nn.Parameter)


_is_compiling = compile_ops.is_compiling


def _grad_safe(*tensors: Any) -> bool:
    """No backward can run through this call: inference mode, grad mode off, or no tensor
    argument that requires grad (the reference's eligibility rule, _dispatch.py:528-553)."""
    if not torch.is_grad_enabled() or (_HAS_INFERENCE_MODE and torch.is_inference_mode_enabled()):
        return True
    return not any(isinstance(t, torch.Tensor) and t.requires_grad for t in tensors)


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
    """Point target.name at wrapper; the first original seen is kept for _restore."""
    _ORIGINALS.setdefault((target, name), getattr(target, name))
    if target is F:
        _STOCK_F[name] = _ORIGINALS[(target, name)]
    setattr(target, name, wrapper)


def _restore(target: Any, name: str) -> None:
    """Put back the original of target.name, if _install replaced it."""
    if (target, name) in _ORIGINALS:
        setattr(target, name, _ORIGINALS.pop((target, name)))


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
        idx = _native.variant_index(op, name[len(_NATIVE_PREFIX):])
    except RuntimeError:
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
    channels-last when `cl_out`.  The conversions run on the native transpose kernel.  A
    channels-last input first goes to the MFMA tiles that stage channels-last patches
    directly (no conversions); shapes they decline take the conversions."""

    def run(i, w, b, s, p, d, variant: int = -1):
        if cl_out:
            try:
                return _native.conv_channels_last(i, w, b, s, p, d, nd, variant=variant)
            except _native.Unsupported:
                pass
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


def _conv_grads(grad_output, input, weight, bias_sizes, conf, needs, fwd):
    """(dx, dw, db) of a patched conv for `needs` = [dx, dw, db] wanted:
    * dx of a stride-1, dilation-1, groups-1 conv through `fwd` (the accelerated forward) on dy
      with transposed, flipped weights;
    * dw of a 'same' 3x3(x3) conv in a 16-bit type through the native wgrad kernel;
    * db as a reduction of dy once every other gradient is native;
    * whatever is left through aten.convolution_backward, the op autograd uses unpatched."""
    stride, padding, dilation, groups, nd = conf
    needs = list(needs)
    gi = gw = gb = None
    if needs[0] and input.is_cuda:
        pad_t = _dgrad_padding(weight, stride, padding, dilation, groups, nd)
        if pad_t is not None:
            gi = _dgrad_via_forward(grad_output, weight.detach(), pad_t, nd, fwd)
            if tuple(gi.shape) == tuple(input.shape):
                needs[0] = False
            else:
                gi = None
    if needs[1] and input.is_cuda:
        gw = _wgrad_native(input, grad_output, weight, stride, padding, dilation, groups, nd)
        if gw is not None:
            needs[1] = False
    if needs[2] and not needs[0] and not needs[1]:
        gb = grad_output.sum(dim=[0] + list(range(2, 2 + nd)), dtype=torch.float32).to(weight.dtype)
        needs[2] = False
    if any(needs):
        tup = _triple if nd == 3 else _pair
        ai, aw, ab = torch.ops.aten.convolution_backward(
            grad_output.contiguous(), input, weight, bias_sizes, list(tup(stride)),
            list(tup(padding)), list(tup(dilation)), False, [0] * nd, groups, needs)
        gi = ai if gi is None else gi
        gw = aw if gw is None else gw
        gb = ab if gb is None else gb
    return gi, gw, gb


class _ConvFn(torch.autograd.Function):
    """Accelerated forward; the backward of _conv_grads (native input and weight gradients
    where they apply, aten.convolution_backward for the rest -- the reference's _Conv3dFn,
    _dispatch.py:2029-2075, uses aten for all of it)."""

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
        needs = [bool(ctx.needs_input_grad[0]), bool(ctx.needs_input_grad[1]),
                 ctx.bias_sizes is not None and bool(ctx.needs_input_grad[2])]
        if not any(needs):
            return (None,) * 9
        gi, gw, gb = _conv_grads(grad_output, input, weight, ctx.bias_sizes, ctx.conf, needs, ctx.fwd)
        return gi, gw, gb, None, None, None, None, None, None


def _stock_conv(nd: int) -> Callable:
    """The unpatched F.conv2d / F.conv3d."""
    return _STOCK_F["conv%dd" % nd]


def _conv_selected(nd: int, input, weight, bias, stride, padding, dilation):
    """Eager body of the conv custom ops: the per-shape selection of the patched API."""
    orig = _stock_conv(nd)
    return _conv_accelerated_forward(nd, input, weight, bias, stride, padding, dilation, 1, orig)


def _conv_grads_eager(grad_output, input, weight, has_bias, stride, padding, dilation, nd, needs):
    """Eager body of the conv backward custom op."""
    orig = _stock_conv(nd)

    def fwd(i, w, b, s, p, d, g):
        return _conv_accelerated_forward(nd, i, w, b, s, p, d, g, orig)
    bias_sizes = [weight.shape[0]] if has_bias else None
    return _conv_grads(grad_output, input, weight, bias_sizes, (stride, padding, dilation, 1, nd),
                       needs, fwd)


def _traced_conv(nd: int, input, weight, bias, stride, padding, dilation, groups, orig):
    """Under torch.compile: an eligible conv becomes one custom-op node (its body selects the
    kernel when the graph runs; autograd included), anything else the stock conv."""
    ok = (groups == 1 and not isinstance(padding, str)
          and isinstance(input, torch.Tensor) and isinstance(weight, torch.Tensor)
          and input.dim() == nd + 2 and weight.dim() == nd + 2
          and input.is_contiguous() and weight.is_contiguous()
          and _usable(input, weight, bias, dtypes=_CONV_NATIVE_DTYPES)
          and input.dtype == weight.dtype and (bias is None or bias.dtype == input.dtype)
          and compile_ops.native_loaded())
    if not ok:
        return orig(input, weight, bias, stride, padding, dilation, groups)
    op = compile_ops.conv3d_native if nd == 3 else compile_ops.conv2d_native
    return op(input, weight, bias, stride, padding, dilation)


def _patched_conv2d(input, weight, bias=None, stride=1, padding=0, dilation=1, groups=1):
    orig = _STOCK_F["conv2d"]
    if _is_compiling():
        if (isinstance(weight, torch.Tensor) and weight.dim() == 4 and not isinstance(padding, str)
                and _is_pointwise_conv2d(weight, stride, padding, dilation)):
            return orig(input, weight, bias, stride, padding, dilation, groups)
        return _traced_conv(2, input, weight, bias, stride, padding, dilation, groups, orig)
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
    orig = _STOCK_F["conv3d"]
    if _is_compiling():
        return _traced_conv(3, input, weight, bias, stride, padding, dilation, groups, orig)

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
    """Native GroupNorm: the named variant, or the first one that accepts the shape."""
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
    orig = _STOCK_F["group_norm"]
    channels_last = isinstance(input, torch.Tensor) and _channels_last(input)
    if channels_last:
        return _group_norm_channels_last(input, num_groups, weight, bias, eps, orig)
    if not (isinstance(input, torch.Tensor) and input.dim() >= 2 and input.is_contiguous()
            and _usable(input, dtypes=_GROUPNORM_DTYPES)
            and _usable(weight, bias, dtypes=_GROUPNORM_DTYPES)
            and isinstance(num_groups, int) and num_groups > 0
            and input.shape[1] % num_groups == 0 and _native.available()):
        if _DEBUG:
            _debug("group_norm", "stock", "layout/dtype outside this tier", input=input)
        return orig(input, num_groups, weight, bias, eps)
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


def _group_norm_grads(grad_output, input, num_groups, weight, eps, needs):
    """(dx, dgamma, dbeta) of GroupNorm for `needs` = (dx, dgamma, dbeta) wanted: the native
    backward kernels for contiguous or channels-last GPU input (channels-last first on the
    channels-last kernels, else through NC[S] copies made by the native transpose, dx coming
    back in the input's layout; dgamma / dbeta in fp32), the textbook torch-op backward
    otherwise (dgamma / dbeta in the parameter dtypes).  Entries not asked for are None."""
    cl = _channels_last(input)
    if input.is_cuda and cl and _native.available():
        try:  # straight on the channels-last layout
            fmt = torch.channels_last if input.dim() == 4 else torch.channels_last_3d
            dy = grad_output if _channels_last(grad_output) else grad_output.contiguous(memory_format=fmt)
            return _native.group_norm_cl_backward(dy, input.detach(), num_groups,
                                                  None if weight is None else weight.detach(), eps, needs)
        except _native.Unsupported:
            pass
    if input.is_cuda and (input.is_contiguous() or cl) and _native.available():
        try:
            x = _native.channels_last_to_contiguous(input.detach()) if cl else input.detach()
            gx, gw, gb = _native.group_norm_backward(_to_ncdhw(grad_output), x, num_groups,
                                                     None if weight is None else weight.detach(),
                                                     eps, needs)
            if cl and gx is not None:
                gx = _native.contiguous_to_channels_last(gx)
            return gx, gw, gb
        except _native.Unsupported:
            pass
    return _group_norm_backward(grad_output.contiguous(), input, num_groups, weight, eps, needs)


class _GroupNormFn(torch.autograd.Function):
    """Accelerated forward; the backward of _group_norm_grads (native kernels where they
    apply; the reference's _GroupNormFn, 2305-2359, uses the torch-op formula)."""

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
        gx, gw, gb = _group_norm_grads(grad_output, input, ctx.num_groups, weight, ctx.eps, needs)
        gw = None if gw is None else gw.to(weight.dtype)
        gb = None if gb is None else gb.to(ctx.bias_dtype if ctx.bias_dtype is not None else input.dtype)
        return gx, gw, gb, None, None


def _traced_group_norm(input, num_groups, weight, bias, eps, orig):
    """Under torch.compile: an eligible GroupNorm becomes one custom-op node (selection at run
    time, native backward through the op's autograd formula), anything else stock."""
    ok = (isinstance(input, torch.Tensor) and input.dim() >= 2
          and (input.is_contiguous() or _channels_last(input))
          and _usable(input, dtypes=_GROUPNORM_DTYPES) and _usable(weight, bias, dtypes=_GROUPNORM_DTYPES)
          and isinstance(num_groups, int) and num_groups > 0 and input.shape[1] % num_groups == 0
          and compile_ops.native_loaded())
    if not ok:
        return orig(input, num_groups, weight, bias, eps)
    return compile_ops.group_norm(input, num_groups, weight, bias, eps)


def _patched_group_norm(input, num_groups, weight=None, bias=None, eps=1e-5):
    if _is_compiling():
        return _traced_group_norm(input, num_groups, weight, bias, eps, _STOCK_F["group_norm"])
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
            return conv_fusion_ops.FusedConvGroupNormSiLU.forward_parts(conv, norm, input)
    return _SEQ_FORWARD_ORIG(self, input)


# ---------------------------------------------------------------------------
# enable / disable (reference _dispatch.py:2913-3050): the functional entry points, the
# Sequential fusion when conv fusion is available, conv3d where torch has it.
# ---------------------------------------------------------------------------
def _patch_table() -> "list[tuple[Any, str, Callable]]":
    table = [(F, "group_norm", _patched_group_norm), (F, "conv2d", _patched_conv2d)]
    if conv_fusion_ops.enabled():
        table.append((torch.nn.Sequential, "forward", _patched_sequential_forward))
    if hasattr(F, "conv3d"):
        table.append((F, "conv3d", _patched_conv3d))
    return table


def enable() -> None:
    """Patch torch.nn.functional so eligible calls route through amd_tuned_torch (idempotent)."""
    global _ENABLED, _SEQ_FORWARD_ORIG
    if _ENABLED:
        if _DEBUG:
            _debug("enable", "noop", "already enabled")
        return
    if _DEBUG:
        _debug("enable", "backends", "", native=_native.available(),
               kernel_select=kernel_select.enabled(), conv_fusion=conv_fusion_ops.enabled())
    table = _patch_table()
    compile_ops.keep_traceable([wrapper for _, _, wrapper in table])
    for target, name, wrapper in table:
        _install(target, name, wrapper)
    _SEQ_FORWARD_ORIG = _ORIGINALS.get((torch.nn.Sequential, "forward"), _SEQ_FORWARD_ORIG)
    _ENABLED = True
    if _DEBUG:
        _debug("enable", "installed", "", patched=",".join(sorted(n for _, n in _ORIGINALS)))


def disable() -> None:
    """Restore every function enable() patched."""
    global _ENABLED
    if _DEBUG:
        _debug("disable", "restored", "", patched=",".join(sorted(n for _, n in _ORIGINALS)))
    for target, name in list(_ORIGINALS):
        _restore(target, name)
    _ENABLED = False


def is_enabled() -> bool:
    return _ENABLED


# ---------------------------------------------------------------------------
# TorchScript guard (reference 3099-3155): a scripted or traced graph cannot call these
# Python wrappers, so torch.jit.script / torch.jit.trace run with the stock functions in
# place and the patches come back afterwards.  Installed at import time.
# ---------------------------------------------------------------------------
@contextlib.contextmanager
def _stock_functions():
    """Lift every patch for the duration of the block (nothing to do when not enabled)."""
    lifted = _ENABLED
    if lifted:
        disable()
    try:
        yield
    finally:
        if lifted:
            enable()


def _jit_under_stock(jit_fn: Callable) -> Callable:
    """jit_fn run inside _stock_functions().  Class scripting resolves names a given number
    of frames above torch.jit.script (its `_frames_up` argument); this wrapper is one more
    frame between the user and jit_fn, so that count is raised by one."""
    params = inspect.signature(jit_fn).parameters
    shifts_frames = "_frames_up" in params

    @functools.wraps(jit_fn)
    def entry(*args, **kwargs):
        if shifts_frames:
            bound = inspect.signature(jit_fn).bind(*args, **kwargs)
            bound.arguments["_frames_up"] = bound.arguments.get("_frames_up", 0) + 1
            args, kwargs = bound.args, bound.kwargs
        with _stock_functions():
            return jit_fn(*args, **kwargs)
    return entry


_ORIG_JIT_SCRIPT = torch.jit.script
_ORIG_JIT_TRACE = torch.jit.trace
_script_with_stock_ops = _jit_under_stock(_ORIG_JIT_SCRIPT)
_trace_with_stock_ops = _jit_under_stock(_ORIG_JIT_TRACE)
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
