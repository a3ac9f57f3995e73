"""Candidate ``merge_attn_states`` / ``MergeAttnStates`` for
fastkernels/tasks/baseline/L1/merge_attn_states.py:30-122.

``merge_attn_states(output, prefix_output, prefix_lse, suffix_output, suffix_lse,
output_lse=None, prefill_tokens_with_context=None, output_scale=None)`` writes the
log-sum-exp merge of two partial attention results into ``output`` (and
``output_lse``) in place; ``MergeAttnStates().forward`` has the reference's
signature.  An fp8 output (``output_scale``) is not supported and raises.
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
    if output_scale is not None:
        raise NotImplementedError("merge_attn_states (gfx950): fp8 output is not supported")
    if torch.compiler.is_compiling() and prefill_tokens_with_context is None:
        torch.ops.fastkernels_amd.merge_attn_states(output, prefix_output, prefix_lse,
                                                    suffix_output, suffix_lse, output_lse)
    else:
        ops.merge_attn_states(output, prefix_output, prefix_lse, suffix_output, suffix_lse,
                              output_lse, prefill_tokens_with_context)


class MergeAttnStates(nn.Module):
    """Online softmax merge of two attention partitions."""

    def forward(self, output: torch.Tensor, prefix_output: torch.Tensor,
                prefix_lse: torch.Tensor, suffix_output: torch.Tensor, suffix_lse: torch.Tensor,
                output_lse: torch.Tensor | None = None) -> None:
        merge_attn_states(output=output, prefix_output=prefix_output, prefix_lse=prefix_lse,
                          suffix_output=suffix_output, suffix_lse=suffix_lse,
                          output_lse=output_lse)
