"""Candidate ``SiluAndMul`` for fastkernels/tasks/baseline/L1/silu_and_mul.py:14-35.

``forward(x)`` returns ``silu(x[..., :d]) * x[..., d:]`` as a new tensor of
shape ``x.shape[:-1] + (d,)``; the activation is rounded to x's dtype before
the product, as in the reference's ``forward_native`` (silu_and_mul.py:19-22).
"""
from __future__ import annotations

import sys
from pathlib import Path

import torch
import torch.nn as nn

try:
    import fastkernels_amd  # noqa: F401
except ImportError:  # loaded by file path from the reference harness
    sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
from fastkernels_amd import ops


class SiluAndMul(nn.Module):
    def __init__(self):
        super().__init__()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        d = x.shape[-1] // 2
        if x.stride(-1) != 1:
            x = x.contiguous()
        out = torch.empty(x.shape[:-1] + (d,), dtype=x.dtype, device=x.device)
        if torch.compiler.is_compiling():
            torch.ops.fastkernels_amd.silu_and_mul(out, x)
        else:
            ops.silu_and_mul(out, x)
        return out
