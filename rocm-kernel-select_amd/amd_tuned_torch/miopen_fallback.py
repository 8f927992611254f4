"""The F.conv1d patch: depthwise/causal conv1d through the gfx950 kernel, stock otherwise.

Interface and call order of the reference's miopen_fallback (amd_tuned_torch/
miopen_fallback.py:229-519): `enable_conv1d_fallback` / `disable_conv1d_fallback` /
`is_conv1d_fallback_enabled`, installed at IMPORT time (independent of enable()) unless
AMD_TUNED_TORCH_MIOPEN_CONV1D_FALLBACK=0; the wrapper tries, in order,

  1. the causal fast path -- only with AMD_TUNED_TORCH_CAUSAL_CONV1D_TRUNCATE=1, which
     reproduces the reference's behaviour of returning the already-truncated length-L
     output for `F.conv1d(x, w, b, padding=K-1, groups=C)` with K in 2..4
     (miopen_fallback.py:81-97,273-309).  By default this package keeps stock's output
     shape (L + K - 1) and such calls go through the depthwise contest below, so the
     result of `[..., :L]` is identical either way;
  2. the depthwise contest: `kernel_select.pick("conv1d", ...)` over this package's
     depthwise kernel variants and stock, with the reference's conv1d verification bar
     (fftconv_ops.py:861-886 -- the bar its depthwise/stock contest uses);
  3. stock F.conv1d, retried after torch.cuda.empty_cache() and finally run on the CPU in
     fp32 when MIOpen reports a `miopenStatus` failure (miopen_fallback.py:434-485).

Depthwise eligibility is wider than the reference's (which required an odd width): any
width <= 64 and padding <= 64, since one kernel serves symmetric and causal padding.
"""
from __future__ import annotations

import os
from typing import Any, Callable, Optional

import torch

from . import _native
from . import compile_ops
from . import depthwise_conv1d_ops
from . import kernel_select

_HAS_INFERENCE_MODE = hasattr(torch, "is_inference_mode_enabled")
_PLAIN_TENSOR_TYPES = (torch.Tensor, torch.nn.Parameter)
_DTYPES = (torch.float16, torch.bfloat16, torch.float32)

# (rtol, atol) of the conv1d contest (reference fftconv_ops.py:861-867)
_CONV1D_TOLERANCES = {
    torch.float16: (2e-2, 2e-2),
    torch.bfloat16: (3e-2, 3e-2),
    torch.float32: (1e-3, 1e-4),
}
_CONV1D_DEFAULT_TOLERANCE = (1e-3, 1e-4)


def _env_flag(name: str, default: str = "0") -> bool:
    return os.environ.get(name, default).strip().lower() not in ("0", "", "false", "no", "off")


_CAUSAL_TRUNCATE = _env_flag("AMD_TUNED_TORCH_CAUSAL_CONV1D_TRUNCATE", "0")


def conv1d_tolerance(dtype: torch.dtype):
    return _CONV1D_TOLERANCES.get(dtype, _CONV1D_DEFAULT_TOLERANCE)


def _grad_safe(*tensors: Any) -> bool:
    if _HAS_INFERENCE_MODE and torch.is_inference_mode_enabled():
        return True
    if not torch.is_grad_enabled():
        return True
    return not any(isinstance(t, torch.Tensor) and t.requires_grad for t in tensors)


def _is_plain_tensor(t: Any) -> bool:
    return not isinstance(t, torch.Tensor) or type(t) in _PLAIN_TENSOR_TYPES


def _scalar(v: Any) -> Any:
    return v[0] if isinstance(v, (tuple, list)) else v


def causal_conv1d_available() -> bool:
    return _native.available()


def _depthwise_shape_ok(input, weight, stride, dilation, groups) -> bool:
    if not (isinstance(input, torch.Tensor) and isinstance(weight, torch.Tensor)
            and input.is_cuda and input.dim() == 3 and weight.dim() == 3):
        return False
    dim = input.shape[1]
    out_ch, in_per_group, width = weight.shape
    if groups != dim or out_ch != dim or in_per_group != 1:
        return False
    return _scalar(stride) == 1 and _scalar(dilation) == 1 and 1 <= width <= depthwise_conv1d_ops.KMAX


def _is_causal_conv1d_eligible(input, weight, stride, padding, dilation, groups) -> bool:
    """Depthwise, width 2..4, padding == width - 1 (miopen_fallback.py:273-291)."""
    if not _depthwise_shape_ok(input, weight, stride, dilation, groups):
        return False
    width = weight.shape[2]
    pad = _scalar(padding)
    return 2 <= width <= 4 and isinstance(pad, int) and pad == width - 1


def _resolve_padding(padding, width: int, length: int):
    """(pad_left, l_out) for F.conv1d's padding argument at stride = dilation = 1, or None."""
    if isinstance(padding, str):
        if padding == "valid":
            return 0, length - width + 1
        if padding == "same":
            return (width - 1) // 2, length
        return None
    p = _scalar(padding)
    if not isinstance(p, int) or p < 0 or p > depthwise_conv1d_ops.PADMAX:
        return None
    return p, length + 2 * p - width + 1


def _is_depthwise_conv1d_eligible(input, weight, bias, stride, padding, dilation, groups) -> bool:
    if not _depthwise_shape_ok(input, weight, stride, dilation, groups):
        return False
    if not all(_is_plain_tensor(t) for t in (input, weight, bias)):
        return False
    if input.dtype not in _DTYPES or weight.dtype != input.dtype:
        return False
    if bias is not None and (not bias.is_cuda or bias.dtype != input.dtype):
        return False
    if not input.is_contiguous():
        return False
    r = _resolve_padding(padding, weight.shape[2], input.shape[2])
    return r is not None and r[1] > 0


class _DwConv1dFn(torch.autograd.Function):
    """Native forward; native backward where the library serves it (input gradient through
    the forward kernel with reversed weights when pad_left <= K-1, weight and bias gradients
    through the streaming reduction kernel when K <= 5), stock aten.convolution_backward for
    the rest."""

    @staticmethod
    def forward(ctx, input, weight, bias, pad_left, l_out, variant):
        ctx.save_for_backward(input, weight)
        ctx.has_bias = bias is not None
        ctx.pad_left, ctx.l_out = pad_left, l_out
        return _native.dwconv1d(input, weight.squeeze(1), bias, pad_left, l_out, variant=variant)

    @staticmethod
    def backward(ctx, dout):
        input, weight = ctx.saved_tensors
        C, _, K = weight.shape
        L = input.shape[-1]
        needs = [bool(ctx.needs_input_grad[0]), bool(ctx.needs_input_grad[1]),
                 ctx.has_bias and bool(ctx.needs_input_grad[2])]
        gi = gw = gb = None
        if dout.is_cuda and _native.available():
            dout = dout.contiguous()
            x = input.detach()
            if needs[0]:
                try:  # dx with dw / db, one pass over x and dout where the fused kernel applies
                    gi, dw32, db32 = _native.dwconv1d_backward(dout, x, weight.detach(), ctx.pad_left,
                                                               (True, needs[1], needs[2]))
                    needs[0] = False
                    if dw32 is not None:
                        gw, needs[1] = dw32.to(weight.dtype).view(C, 1, K), False
                    if db32 is not None:
                        gb, needs[2] = db32.to(dout.dtype), False
                except _native.Unsupported:
                    pass
            if needs[1] or needs[2]:
                try:
                    _, dw32, db32 = _native.dwconv1d_backward(dout, x, weight.detach(), ctx.pad_left,
                                                              (False, needs[1], needs[2]))
                    gw = None if dw32 is None else dw32.to(weight.dtype).view(C, 1, K)
                    gb = None if db32 is None else db32.to(dout.dtype)
                    needs[1] = needs[2] = False
                except _native.Unsupported:
                    pass
            if not any(needs):
                return gi, gw, gb, None, None, None
        sgi, sgw, sgb = _DwConv1dFn._stock_backward(ctx, dout, input, weight, needs)
        return (gi if gi is not None else sgi, gw if gw is not None else sgw,
                gb if gb is not None else sgb, None, None, None)

    @staticmethod
    def _stock_backward(ctx, dout, input, weight, needs):
        C, _, K = weight.shape
        L = input.shape[-1]
        # stock semantics of a left-pad / right-crop: pad so the stock conv spans l_out
        pad_right = ctx.l_out - (L + ctx.pad_left - K + 1)
        xin = torch.nn.functional.pad(input.detach(), (ctx.pad_left, max(0, pad_right)))
        if pad_right < 0:
            xin = xin[..., :xin.shape[-1] + pad_right]
        gi, gw, gb = torch.ops.aten.convolution_backward(
            dout.contiguous(), xin, weight, [C] if ctx.has_bias else None, [1], [0], [1], False,
            [0], C, needs)
        if gi is not None:
            gi = gi[..., ctx.pad_left:ctx.pad_left + L]
            if gi.shape[-1] < L:
                gi = torch.nn.functional.pad(gi, (0, L - gi.shape[-1]))
        return gi, gw, gb


def _dw_call(input, weight, bias, pad_left, l_out, variant):
    if _grad_safe(input, weight, bias):
        # the [C, 1, K] weight as it is: the same memory as [C, K]
        return _native.dwconv1d(input, weight, bias, pad_left, l_out, variant=variant)
    return _DwConv1dFn.apply(input, weight, bias, pad_left, l_out, variant)


def _dw_candidates(input, weight, bias, pad_left, l_out) -> list:
    out = []
    for i, name in enumerate(_native.variants(_native.OP_DWCONV1D)):
        def thunk(i=i):
            try:
                return _dw_call(input, weight, bias, pad_left, l_out, i)
            except _native.Unsupported:
                return None
        out.append(("native." + name, thunk))
    return out


def _try_causal_conv1d_fastpath(input, weight, bias, stride, padding, dilation, groups):
    """Reference-shape causal path (length-L output); active only with
    AMD_TUNED_TORCH_CAUSAL_CONV1D_TRUNCATE=1."""
    if not _CAUSAL_TRUNCATE or not _native.available():
        return None
    if not (_is_causal_conv1d_eligible(input, weight, stride, padding, dilation, groups)
            and _is_depthwise_conv1d_eligible(input, weight, bias, stride, padding, dilation,
                                              groups)):
        return None
    try:
        return _dw_call(input, weight, bias, weight.shape[2] - 1, input.shape[2], -1)
    except RuntimeError:
        return None


def _try_depthwise_fastpath(input, weight, bias, stride, padding, dilation, groups,
                            orig_fn: Callable) -> Optional[torch.Tensor]:
    """One contest over {native depthwise variants, stock} keyed like every conv contest."""
    if not (_native.available()
            and _is_depthwise_conv1d_eligible(input, weight, bias, stride, padding, dilation,
                                              groups)):
        return None
    pad_left, l_out = _resolve_padding(padding, weight.shape[2], input.shape[2])
    if kernel_select.enabled():
        won = kernel_select.cached("conv1d", input, weight, stride, padding, dilation)
        if won == "stock":
            return orig_fn(input, weight, bias, stride, padding, dilation, groups)
        if won is not None and won.startswith("native."):
            try:
                vi = _native.variant_index(_native.OP_DWCONV1D, won[7:])
            except RuntimeError:
                vi = None
            if vi is not None:
                try:
                    return _dw_call(input, weight, bias, pad_left, l_out, vi)
                except _native.Unsupported:
                    pass
        candidates = _dw_candidates(input, weight, bias, pad_left, l_out)
        candidates.append(("stock", lambda: orig_fn(input, weight, bias, stride, padding,
                                                    dilation, groups)))
        return kernel_select.pick("conv1d", input, weight, stride, padding, dilation, candidates,
                                  tolerance=conv1d_tolerance(input.dtype))
    try:
        return _dw_call(input, weight, bias, pad_left, l_out, -1)
    except _native.Unsupported:
        return None


def _is_channel_last(x) -> bool:
    """(B, D, L) with unit channel stride: the layout causal_conv1d_fn treats as channel-last
    (src/causal-conv1d-amd/csrc/causal_conv1d.cpp:156)."""
    return isinstance(x, torch.Tensor) and x.dim() == 3 and x.stride(1) == 1 and x.stride(2) > 1


def _try_channel_last_fastpath(input, weight, bias, stride, padding, dilation, groups):
    """Depthwise conv1d on a channel-last x: the channels-last kernel through the BLH op on
    transposed views (native forward and backward), output in the same channel-last layout
    causal_conv1d_fn returns.  None (-> stock) outside that kernel's shapes."""
    if not (_native.available() and _is_channel_last(input) and input.is_cuda
            and _depthwise_shape_ok(input, weight, stride, dilation, groups)
            and all(_is_plain_tensor(t) for t in (input, weight, bias))
            and input.dtype in _DTYPES and weight.dtype == input.dtype
            and (bias is None or (bias.is_cuda and bias.dtype == input.dtype))):
        return None
    if isinstance(padding, str):
        return None
    r = _resolve_padding(padding, weight.shape[2], input.shape[2])
    if r is None or r[1] <= 0:
        return None
    pad = r[0]
    D = input.shape[1]
    w_kd = weight.squeeze(1).t()  # [K, D], the BLH weight layout
    b = bias if bias is not None else torch.zeros(D, dtype=input.dtype, device=input.device)
    try:
        if _grad_safe(input, weight, bias):
            y = depthwise_conv1d_ops.conv1d_forward(input.transpose(1, 2), w_kd, b, pad, False)
        else:
            y = depthwise_conv1d_ops.DepthwiseConv1dFn.apply(input.transpose(1, 2), w_kd, b, pad, False)
    except _native.Unsupported:
        return None
    return y.transpose(1, 2)


def _traced_conv1d(input, weight, bias, stride, padding, dilation, groups, orig_fn):
    """Under torch.compile: a (B, C, L) depthwise conv with integer padding becomes the
    `amd_tuned_torch::depthwise_conv1d_forward` node (with its backward op under autograd);
    anything else is the stock conv, which Dynamo traces as usual."""
    pad = _scalar(padding)
    ok = (compile_ops.native_loaded() and isinstance(pad, int) and not isinstance(pad, bool)
          and _is_depthwise_conv1d_eligible(input, weight, bias, stride, padding, dilation, groups))
    if not ok:
        return orig_fn(input, weight, bias, stride, padding, dilation, groups)
    w = weight.squeeze(1)
    b = bias if bias is not None else input.new_zeros((weight.shape[0],))
    # (inference mode cannot be queried while tracing; grad mode and requires_grad can)
    if not (torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (input, weight, bias))):
        return depthwise_conv1d_ops.conv1d_forward(input, w, b, pad, True)
    return depthwise_conv1d_ops.DepthwiseConv1dFn.apply(input, w, b, pad, True)


def _is_miopen_failure(exc: BaseException) -> bool:
    return isinstance(exc, RuntimeError) and "miopenStatus" in str(exc)


def _stock_with_rescue(op_name: str, orig_fn: Callable, input, weight, bias, stride, padding,
                       dilation, groups):
    """The stock conv, rescued from MIOpen failures the way the reference's wrapper does
    (miopen_fallback.py:434-485): a GPU call that fails with a `miopenStatus` error is tried
    once more after torch.cuda.empty_cache() (MIOpen's workspace allocation is the usual
    cause), and if that fails too the conv runs on the CPU in fp32 and the result comes back
    to the input's device and dtype.  Every other error propagates."""
    attempts = 2 if input.is_cuda else 1
    for attempt in range(attempts):
        if attempt:
            torch.cuda.empty_cache()
        try:
            return orig_fn(input, weight, bias, stride, padding, dilation, groups)
        except RuntimeError as exc:
            if not _is_miopen_failure(exc):
                raise
    print(f"MIOpen fallback ({op_name}): CPU used for this convolution (slow). "
          f"x shape: {tuple(input.shape)}, weight shape: {tuple(weight.shape)}")
    on_cpu = [None if t is None else t.float().cpu() for t in (input, weight, bias)]
    out = orig_fn(*on_cpu, stride, padding, dilation, groups)
    return out.to(device=input.device, dtype=input.dtype)


def _miopen_safe_conv(op_name: str, orig_fn: Callable) -> Callable:
    """The F.conv1d replacement: the native paths in the reference's order, then stock."""

    def wrapped(input, weight, bias=None, stride=1, padding=0, dilation=1, groups=1):
        if compile_ops.is_compiling():
            return _traced_conv1d(input, weight, bias, stride, padding, dilation, groups, orig_fn)
        args = (input, weight, bias, stride, padding, dilation, groups)
        for fast_path in (_try_causal_conv1d_fastpath, _try_channel_last_fastpath):
            out = fast_path(*args)
            if out is not None:
                return out
        out = _try_depthwise_fastpath(*args, orig_fn)
        if out is not None:
            return out
        return _stock_with_rescue(op_name, orig_fn, *args)

    return wrapped


# The installed wrapper and the F.conv1d it replaced (None while not installed).
_original_conv1d: Optional[Callable] = None


def enable_conv1d_fallback() -> None:
    """Install the F.conv1d wrapper (idempotent)."""
    global _original_conv1d
    if _original_conv1d is None:
        stock = torch.nn.functional.conv1d
        torch.nn.functional.conv1d = _miopen_safe_conv("conv1d", stock)
        _original_conv1d = stock


def disable_conv1d_fallback() -> None:
    """Put stock F.conv1d back (idempotent)."""
    global _original_conv1d
    if _original_conv1d is not None:
        torch.nn.functional.conv1d, _original_conv1d = _original_conv1d, None


def is_conv1d_fallback_enabled() -> bool:
    return _original_conv1d is not None


# Installed at import, independently of enable(); AMD_TUNED_TORCH_MIOPEN_CONV1D_FALLBACK=0
# leaves F.conv1d alone.
if _env_flag("AMD_TUNED_TORCH_MIOPEN_CONV1D_FALLBACK", default="1"):
    enable_conv1d_fallback()
