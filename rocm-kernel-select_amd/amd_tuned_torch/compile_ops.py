"""torch.library custom ops over the accelerated operators, for torch.compile.

While Dynamo traces a model, the patched F.conv2d / F.conv3d / F.group_norm /
group_norm_silu and the depthwise F.conv1d do not run their Python dispatch (a ctypes call
on a fake tensor cannot be traced, and the per-shape contest must not run at trace time).
They emit one of these ops instead: an opaque graph node whose shape comes from the fake
implementation and whose real body runs when the compiled graph runs.  The real body is the
same dispatch the eager API uses: the shape's cached winner, or -- on the first call for a
shape -- the contest among this package's kernel variants and stock.  That is how the
reference's `_C.conv2d` / `_C.conv3d` behave behind the same op names: the native extension
picks its own variant inside the op (src/main_rocm.cpp:408-512,669-715,798-854).

Names, schemas and fakes follow the reference (amd_tuned_torch/compile_ops.py:168-235,
369-415): `amd_tuned_torch::group_norm`, `::conv2d_native`, `::conv3d_native`; the conv fakes
take aten's own conv meta kernels for the output size.  Beyond the reference, the ops carry
autograd formulas -- the GroupNorm and conv backwards are further opaque ops running the
native backward kernels -- so a compiled training step keeps the native path, and
`::group_norm_silu` covers the fused GroupNorm+SiLU.  Eligibility is checked by the caller.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _native


def is_compiling() -> bool:
    """True while Dynamo traces (torch.compile); False in eager code and at graph run time."""
    probe = getattr(getattr(torch, "compiler", None), "is_compiling", None)
    if probe is None:
        probe = getattr(getattr(torch, "_dynamo", None), "is_compiling", None)
    try:
        return bool(probe()) if probe is not None else False
    except Exception:
        return False


def keep_traceable(wrappers) -> None:
    """torch.compile keeps a table of torch functions that it records as opaque calls in the
    graph instead of tracing into them.  The table is built once, by looking the functions up
    by name (torch.nn.functional.group_norm among them), the first time torch._dynamo is
    imported.  Built while a wrapper of this package stands in for such a function, it would
    list the wrapper, and Dynamo would never see the wrapper's compile route.  So the table is
    built now -- before the wrappers go in -- and any wrapper already listed is dropped."""
    try:
        from torch._dynamo import trace_rules
        table = trace_rules.get_torch_obj_rule_map()
    except Exception:  # a torch without Dynamo: nothing to keep in step
        return
    for fn in wrappers:
        table.pop(fn, None)


def _triple(v):
    return (v, v, v) if isinstance(v, int) else tuple(v)


def _pair(v):
    return (v, v) if isinstance(v, int) else tuple(v)


def _placeholder(like: torch.Tensor) -> torch.Tensor:
    """Stands in for a gradient that was not asked for (custom-op outputs cannot be None)."""
    return like.new_empty((0,))


def _conform(t: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    """`t` with the dtype and strides of `like`, which is what a fake built by
    torch.empty_like(like) promised the compiled graph.  The eager bodies can return other
    dtypes (a stock fallback keeps the parameter dtype, a float32 weight promotes the input
    gradient) or layouts; a graph built on the fake would then read the buffer with the wrong
    element size or stride."""
    if t.dtype == like.dtype and t.shape == like.shape and t.stride() == like.stride():
        return t
    out = torch.empty_like(like)
    out.copy_(t)
    return out


def _f32_vector(t: torch.Tensor) -> torch.Tensor:
    """A 1-D float32 contiguous gradient (the GroupNorm backward fake's dgamma / dbeta)."""
    return t.to(torch.float32).contiguous()


# ---------------------------------------------------------------------------
# Eager bodies: the dispatch the patched API runs, reached lazily (the dispatch modules
# import this one).
# ---------------------------------------------------------------------------
def _gn_forward(input_, num_groups, weight, bias, eps):
    from . import _dispatch
    return _dispatch._group_norm_accelerated_forward(input_, num_groups, weight, bias, eps)


def _gn_backward(grad, input_, num_groups, weight, eps, mask):
    from . import _dispatch
    return _dispatch._group_norm_grads(grad, input_, num_groups, weight, eps, tuple(mask))


def _gn_silu_forward(x, num_groups, weight, bias, eps):
    from . import conv_fusion_ops
    return conv_fusion_ops.group_norm_silu(x, num_groups, weight, bias, eps)


def _conv_forward(nd, input_, weight, bias, stride, padding, dilation):
    from . import _dispatch
    return _dispatch._conv_selected(nd, input_, weight, bias, stride, padding, dilation)


def _conv_backward(grad, input_, weight, has_bias, stride, padding, dilation, nd, mask):
    from . import _dispatch
    return _dispatch._conv_grads_eager(grad, input_, weight, has_bias, stride, padding, dilation, nd,
                                       tuple(mask))


def _registered(name: str) -> bool:
    return hasattr(torch.ops, "amd_tuned_torch") and hasattr(torch.ops.amd_tuned_torch, name)


_HAS_CUSTOM_OP = hasattr(torch.library, "custom_op") and hasattr(torch.library, "register_autograd")

if _HAS_CUSTOM_OP and not _registered("group_norm"):
    # --- GroupNorm -------------------------------------------------------------------
    @torch.library.custom_op("amd_tuned_torch::group_norm", mutates_args=())
    def _group_norm_op(input_: torch.Tensor, num_groups: int, weight: Optional[torch.Tensor],
                       bias: Optional[torch.Tensor], eps: float) -> torch.Tensor:
        return _gn_forward(input_, num_groups, weight, bias, eps)

    @_group_norm_op.register_fake
    def _(input_, num_groups, weight, bias, eps):
        return torch.empty_like(input_)  # shape- and memory-format-preserving

    @torch.library.custom_op("amd_tuned_torch::group_norm_backward", mutates_args=())
    def _group_norm_bwd_op(grad: torch.Tensor, input_: torch.Tensor, num_groups: int,
                           weight: Optional[torch.Tensor], eps: float, mask: list[bool]
                           ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        gx, gw, gb = _gn_backward(grad, input_, num_groups, weight, eps, mask)
        # the native backward gives dgamma / dbeta in float32, the torch-op fallback (a shape
        # the native kernels decline) in the parameter dtypes: the fake promises float32
        return (_conform(gx, input_) if gx is not None else _placeholder(input_),
                _f32_vector(gw) if gw is not None else _placeholder(input_),
                _f32_vector(gb) if gb is not None else _placeholder(input_))

    @_group_norm_bwd_op.register_fake
    def _(grad, input_, num_groups, weight, eps, mask):
        C = input_.shape[1]
        return (torch.empty_like(input_) if mask[0] else _placeholder(input_),
                input_.new_empty((C,), dtype=torch.float32) if mask[1] else _placeholder(input_),
                input_.new_empty((C,), dtype=torch.float32) if mask[2] else _placeholder(input_))

    def _gn_setup(ctx, inputs, output):
        input_, num_groups, weight, bias, eps = inputs
        ctx.save_for_backward(input_, weight)
        ctx.num_groups, ctx.eps = num_groups, eps
        ctx.has_weight, ctx.has_bias = weight is not None, bias is not None
        ctx.weight_dtype = weight.dtype if weight is not None else None
        ctx.bias_dtype = bias.dtype if bias is not None else input_.dtype

    def _gn_grad(ctx, grad):
        input_, weight = ctx.saved_tensors
        mask = [bool(ctx.needs_input_grad[0]), ctx.has_weight and bool(ctx.needs_input_grad[2]),
                ctx.has_bias and bool(ctx.needs_input_grad[3])]
        gx, gw, gb = torch.ops.amd_tuned_torch.group_norm_backward(
            grad, input_, ctx.num_groups, weight, ctx.eps, mask)
        return (gx if mask[0] else None, None, gw.to(ctx.weight_dtype) if mask[1] else None,
                gb.to(ctx.bias_dtype) if mask[2] else None, None)

    torch.library.register_autograd("amd_tuned_torch::group_norm", _gn_grad, setup_context=_gn_setup)

    # --- GroupNorm + SiLU (forward only; with a gradient live the caller composes the
    # patched group_norm and F.silu) --------------------------------------------------
    @torch.library.custom_op("amd_tuned_torch::group_norm_silu", mutates_args=())
    def _group_norm_silu_op(input_: torch.Tensor, num_groups: int, weight: Optional[torch.Tensor],
                            bias: Optional[torch.Tensor], eps: float) -> torch.Tensor:
        return _gn_silu_forward(input_, num_groups, weight, bias, eps)

    @_group_norm_silu_op.register_fake
    def _(input_, num_groups, weight, bias, eps):
        return torch.empty_like(input_)

    # --- conv2d / conv3d ---------------------------------------------------------------
    @torch.library.custom_op("amd_tuned_torch::conv2d_native", mutates_args=())
    def _conv2d_native_op(input_: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
                          stride: list[int], padding: list[int], dilation: list[int]) -> torch.Tensor:
        return _conv_forward(2, input_, weight, bias, stride, padding, dilation)

    @_conv2d_native_op.register_fake
    def _(input_, weight, bias, stride, padding, dilation):
        return torch.ops.aten.conv2d.default(input_, weight, bias, stride, padding, dilation, 1)

    @torch.library.custom_op("amd_tuned_torch::conv3d_native", mutates_args=())
    def _conv3d_native_op(input_: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
                          stride: list[int], padding: list[int], dilation: list[int]) -> torch.Tensor:
        return _conv_forward(3, input_, weight, bias, stride, padding, dilation)

    @_conv3d_native_op.register_fake
    def _(input_, weight, bias, stride, padding, dilation):
        return torch.ops.aten.conv3d.default(input_, weight, bias, stride, padding, dilation, 1)

    @torch.library.custom_op("amd_tuned_torch::conv_backward", mutates_args=())
    def _conv_bwd_op(grad: torch.Tensor, input_: torch.Tensor, weight: torch.Tensor, has_bias: bool,
                     stride: list[int], padding: list[int], dilation: list[int], nd: int,
                     mask: list[bool]) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        gi, gw, gb = _conv_backward(grad, input_, weight, has_bias, stride, padding, dilation, nd, mask)
        return (_conform(gi, input_) if gi is not None else _placeholder(input_),
                _conform(gw, weight) if gw is not None else _placeholder(input_),
                gb.to(weight.dtype).contiguous() if gb is not None else _placeholder(input_))

    @_conv_bwd_op.register_fake
    def _(grad, input_, weight, has_bias, stride, padding, dilation, nd, mask):
        return (torch.empty_like(input_) if mask[0] else _placeholder(input_),
                torch.empty_like(weight) if mask[1] else _placeholder(input_),
                weight.new_empty((weight.shape[0],)) if mask[2] else _placeholder(input_))

    def _conv_setup_for(nd):
        def setup(ctx, inputs, output):
            input_, weight, bias, stride, padding, dilation = inputs
            ctx.save_for_backward(input_, weight)
            ctx.conf = (list(stride), list(padding), list(dilation), nd)
            ctx.has_bias = bias is not None
        return setup

    def _conv_grad(ctx, grad):
        input_, weight = ctx.saved_tensors
        stride, padding, dilation, nd = ctx.conf
        mask = [bool(ctx.needs_input_grad[0]), bool(ctx.needs_input_grad[1]),
                ctx.has_bias and bool(ctx.needs_input_grad[2])]
        gi, gw, gb = torch.ops.amd_tuned_torch.conv_backward(grad, input_, weight, ctx.has_bias, stride,
                                                             padding, dilation, nd, mask)
        return (gi if mask[0] else None, gw if mask[1] else None, gb if mask[2] else None,
                None, None, None)

    torch.library.register_autograd("amd_tuned_torch::conv2d_native", _conv_grad,
                                    setup_context=_conv_setup_for(2))
    torch.library.register_autograd("amd_tuned_torch::conv3d_native", _conv_grad,
                                    setup_context=_conv_setup_for(3))

if _HAS_CUSTOM_OP:
    _ops = torch.ops.amd_tuned_torch

    def _group_norm_impl(input_, num_groups, weight, bias, eps):
        return _ops.group_norm(input_, num_groups, weight, bias, eps)

    def _group_norm_silu_impl(input_, num_groups, weight, bias, eps):
        return _ops.group_norm_silu(input_, num_groups, weight, bias, eps)

    def _conv2d_native_impl(input_, weight, bias, stride, padding, dilation):
        return _ops.conv2d_native(input_, weight, bias, stride, padding, dilation)

    def _conv3d_native_impl(input_, weight, bias, stride, padding, dilation):
        return _ops.conv3d_native(input_, weight, bias, stride, padding, dilation)
else:  # torch without custom ops: the same eager bodies, no graph node
    _group_norm_impl = _gn_forward
    _group_norm_silu_impl = _gn_silu_forward

    def _conv2d_native_impl(input_, weight, bias, stride, padding, dilation):
        return _conv_forward(2, input_, weight, bias, stride, padding, dilation)

    def _conv3d_native_impl(input_, weight, bias, stride, padding, dilation):
        return _conv_forward(3, input_, weight, bias, stride, padding, dilation)


def group_norm(input_: torch.Tensor, num_groups: int, weight: Optional[torch.Tensor] = None,
               bias: Optional[torch.Tensor] = None, eps: float = 1e-5) -> torch.Tensor:
    """The accelerated GroupNorm as one graph node (NC[S] or channels-last input)."""
    return _group_norm_impl(input_, num_groups, weight, bias, eps)


def group_norm_silu(input_: torch.Tensor, num_groups: int, weight: Optional[torch.Tensor] = None,
                    bias: Optional[torch.Tensor] = None, eps: float = 1e-5) -> torch.Tensor:
    """SiLU(GroupNorm(x)) as one graph node; forward only."""
    return _group_norm_silu_impl(input_, num_groups, weight, bias, eps)


def conv2d_native(input_, weight, bias=None, stride=1, padding=0, dilation=1) -> torch.Tensor:
    """gfx950 implicit-GEMM conv2d (groups = 1; fp16/bf16/fp32; NCHW) as one graph node."""
    return _conv2d_native_impl(input_, weight, bias, list(_pair(stride)), list(_pair(padding)),
                               list(_pair(dilation)))


def conv3d_native(input_, weight, bias=None, stride=1, padding=0, dilation=1) -> torch.Tensor:
    """gfx950 implicit-GEMM conv3d (groups = 1; fp16/bf16/fp32; NCDHW) as one graph node."""
    return _conv3d_native_impl(input_, weight, bias, list(_triple(stride)),
                               list(_triple(padding)), list(_triple(dilation)))


def native_loaded() -> bool:
    """Whether the kernel library is loaded (a plain flag, safe to read while tracing)."""
    return _native._lib is not None
