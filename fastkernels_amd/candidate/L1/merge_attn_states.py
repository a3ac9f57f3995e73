"""Candidate ``merge_attn_states`` / ``MergeAttnStates`` for
fastkernels/tasks/baseline/L1/merge_attn_states.py:30-122.

``merge_attn_states(output, prefix_output, prefix_lse, suffix_output, suffix_lse,
output_lse=None, prefill_tokens_with_context=None, output_scale=None)`` writes the
log-sum-exp merge of two partial attention results into ``output`` (and
``output_lse``) in place; ``MergeAttnStates().forward`` has the reference's
signature.  A float8_e4m3fn ``output`` takes ``output_scale`` (one float32 value):
the merged (or copied) values are divided by it, clamped to +-448 and rounded to
e4m3fn, as the reference's USE_FP8_OUTPUT form (merge_attn_states.cu:2436-2571).
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


def merge_attn_states(output: torch.Tensor, prefix_output: torch.Tensor,
                      prefix_lse: torch.Tensor, suffix_output: torch.Tensor,
                      suffix_lse: torch.Tensor, output_lse: torch.Tensor | None = None,
                      prefill_tokens_with_context: int | None = None,
                      output_scale: torch.Tensor | None = None) -> None:
    if output.dtype not in (torch.float32, torch.half, torch.bfloat16) and output_scale is None:
        raise ValueError(f"output_scale is required when output is {output.dtype}")
    if output_scale is not None and output.dtype in (torch.float32, torch.half, torch.bfloat16):
        output_scale = None  # only an fp8 output is scaled
    if output_scale is not None and (output_scale.dtype != torch.float32 or
                                     output_scale.device != output.device):
        output_scale = output_scale.to(device=output.device, dtype=torch.float32)
    if torch.compiler.is_compiling():
        torch.ops.fastkernels_amd.merge_attn_states(output, prefix_output, prefix_lse,
                                                    suffix_output, suffix_lse, output_lse,
                                                    prefill_tokens_with_context, output_scale)
    else:
        ops.merge_attn_states(output, prefix_output, prefix_lse, suffix_output, suffix_lse,
                              output_lse, prefill_tokens_with_context, output_scale)


class MergeAttnStates(nn.Module):
    """Online softmax merge of two attention partitions."""

    def forward(self, output: torch.Tensor, prefix_output: torch.Tensor,
                prefix_lse: torch.Tensor, suffix_output: torch.Tensor, suffix_lse: torch.Tensor,
                output_lse: torch.Tensor | None = None) -> None:
        merge_attn_states(output=output, prefix_output=prefix_output, prefix_lse=prefix_lse,
                          suffix_output=suffix_output, suffix_lse=suffix_lse,
                          output_lse=output_lse)
