"""amd_tuned_torch for MI355X (gfx950).

`import amd_tuned_torch` patches torch.nn.functional so that depthwise/causal conv1d,
conv2d, conv3d and GroupNorm (plus the GroupNorm+SiLU of nn.Sequential(GroupNorm, SiLU,
Conv2d)) run through hand-written gfx950 kernels whenever a per-shape, first-call
benchmark says they beat stock PyTorch -- the import surface of the reference package
(amd_tuned_torch/__init__.py:513-610): enable() at import unless
AMD_TUNED_TORCH_AUTOPATCH=0, the F.conv1d wrapper installed at import independently of
enable(), and the selector / dispatch / fusion modules re-exported.

The kernels live in one C-ABI library (amd_tuned_torch/_lib/libamd_tuned_torch_hip.so,
built by rocm-kernel-select_amd/build_lib.py).  On a machine with a GPU the library is
required: importing without it raises ImportError, so nothing silently falls back.
"""
from __future__ import annotations

import os

import torch

from . import _native

try:
    _native.load()
    _NATIVE_OK = True
except OSError as _exc:  # no library
    _NATIVE_OK = False
    if torch.cuda.device_count() > 0 and os.environ.get("AMD_TUNED_TORCH_ALLOW_NO_NATIVE", "0") == "0":
        raise ImportError(
            "amd_tuned_torch: the gfx950 kernel library is not built/loadable "
            f"({_exc}); run `python rocm-kernel-select_amd/build_lib.py`") from _exc

from . import kernel_select  # noqa: E402
from . import conv_fusion_ops  # noqa: E402
from . import compile_ops  # noqa: E402
from . import depthwise_conv1d_ops  # noqa: E402
from . import causal_conv1d  # noqa: E402
from . import miopen_fallback  # noqa: E402  (installs the F.conv1d wrapper at import)
from . import _dispatch  # noqa: E402
from ._dispatch import *  # noqa: E402,F401,F403
from ._dispatch import enable, disable, is_enabled, ops  # noqa: E402
from .conv_fusion_ops import group_norm_silu, replace_conv_blocks, unfuse_conv_blocks  # noqa: E402

__version__ = "0.1.0"


def native_available() -> bool:
    """True when the kernel library is loaded."""
    return _NATIVE_OK


if os.environ.get("AMD_TUNED_TORCH_AUTOPATCH", "1") != "0":
    enable()
