"""Writes tests/golden/golden.npz: small input/output vectors of the hot-path operators
computed by STOCK torch.nn.functional in float64 on the CPU -- the reference's parity target
(amd_tuned_torch/kernel_select.py:68-82: every candidate is verified against stock).

    python tests/golden/make_golden.py

The reference ships no stored vectors for this path (its numeric tests compare against
stock live), so the fixtures are produced from stock here and committed with this script.
"""
from __future__ import annotations

import os

import numpy as np
import torch
import torch.nn.functional as F

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")


def main() -> None:
    g = torch.Generator().manual_seed(20261201)
    d = torch.float64
    arrs = {}

    def rnd(*s, scale=1.0):
        return torch.randn(*s, generator=g, dtype=d) * scale

    # depthwise conv1d: symmetric (k3 p1), causal stock shape (k4 p3), 'valid' (k5 p0), wide pad
    for name, (N, C, L, K, p) in {"dw_sym": (2, 3, 11, 3, 1), "dw_causal": (2, 3, 9, 4, 3),
                                  "dw_valid": (1, 2, 12, 5, 0), "dw_widepad": (1, 2, 6, 3, 4)}.items():
        x, w, b = rnd(N, C, L), rnd(C, 1, K, scale=K ** -0.5), rnd(C, scale=0.3)
        y = F.conv1d(x, w, b, padding=p, groups=C)
        arrs.update({f"{name}_x": x, f"{name}_w": w, f"{name}_b": b, f"{name}_y": y,
                     f"{name}_meta": torch.tensor([N, C, L, K, p], dtype=torch.int64)})
    # GroupNorm (affine), GroupNorm + SiLU, non-affine 3-D
    x = rnd(2, 6, 4, 5) + torch.linspace(-2, 2, 6, dtype=d).view(1, 6, 1, 1)
    gm, bt = 1 + rnd(6, scale=0.1), rnd(6, scale=0.1)
    arrs.update({"gn_x": x, "gn_g": gm, "gn_b": bt, "gn_y": F.group_norm(x, 3, gm, bt, 1e-5),
                 "gn_silu_y": F.silu(F.group_norm(x, 3, gm, bt, 1e-5))})
    x3 = rnd(1, 4, 3, 2, 5)
    arrs.update({"gn3_x": x3, "gn3_y": F.group_norm(x3, 2, None, None, 1e-6)})
    # conv2d (stride 2, asymmetric pad, dilation) and conv3d (pad 1 / k3, mixed stride)
    x2, w2, b2 = rnd(1, 3, 7, 8), rnd(4, 3, 3, 2, scale=0.3), rnd(4, scale=0.1)
    arrs.update({"c2_x": x2, "c2_w": w2, "c2_b": b2,
                 "c2_y": F.conv2d(x2, w2, b2, stride=(2, 1), padding=(1, 2), dilation=(1, 2))})
    x3c, w3c, b3c = rnd(1, 2, 4, 5, 6), rnd(3, 2, 3, 3, 3, scale=0.3), rnd(3, scale=0.1)
    arrs.update({"c3_x": x3c, "c3_w": w3c, "c3_b": b3c,
                 "c3_y": F.conv3d(x3c, w3c, b3c, stride=(1, 2, 1), padding=1)})
    np.savez(OUT, **{k: v.numpy() for k, v in arrs.items()})
    print("wrote", OUT, len(arrs), "arrays")


if __name__ == "__main__":
    main()
