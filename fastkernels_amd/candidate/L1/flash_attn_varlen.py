"""Candidate ``FlashAttnVarlen`` for fastkernels/tasks/baseline/L1/flash_attn_varlen.py:21-47.

Variable-length attention over dense (no block table) query / key / value tensors:
``forward(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
softmax_scale, causal=True, return_softmax_lse=False)`` with ``q [total_q, Hq, D]``
and ``k`` / ``v`` ``[total_k, Hk, D]`` (rows ``cu_seqlens_k[b] .. cu_seqlens_k[b+1]``
are sequence b's keys; ``Hq`` a multiple of ``Hk``); causal queries are aligned to
the end of their sequence's keys, as in flash_attn_varlen_func.  Returns
``[total_q, Hq, D]`` in q's dtype.  The reference's caller without a KV cache is
the encoder attention (L2/encoder_attention.py:37), bidirectional.

It runs on the same gfx950 kernel as ``FlashAttnPrefill``'s dense path
(``fk_varlen_prefill``): bf16 inputs, head sizes 64, 128 and 256.  What that
kernel does not produce raises ``NotImplementedError`` rather than computing
something else: the softmax log-sum-exp (``return_softmax_lse=True``, used by
the MLA chunked-prefix merge, whose value head size also differs from the query
head size) and query / value head sizes that differ.
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


class FlashAttnVarlen(nn.Module):
    def forward(self, q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                softmax_scale, causal=True, return_softmax_lse=False):
        if return_softmax_lse:
            raise NotImplementedError("FlashAttnVarlen (gfx950): return_softmax_lse is not "
                                      "produced by the dense prefill kernel")
        if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
            raise ValueError("FlashAttnVarlen: q, k, v must be [tokens, heads, head_dim]")
        total, hq, d = q.shape
        if k.shape[2] != d or v.shape[2] != d:
            raise NotImplementedError("FlashAttnVarlen (gfx950): query, key and value head "
                                      f"sizes must match (got {d}, {k.shape[2]}, {v.shape[2]})")
        if cu_seqlens_q.dtype != torch.int32:
            cu_seqlens_q = cu_seqlens_q.to(torch.int32)
        if cu_seqlens_k.dtype != torch.int32:
            cu_seqlens_k = cu_seqlens_k.to(torch.int32)
        out = torch.empty((total, hq, d), dtype=q.dtype, device=q.device)
        # A bound on every sequence's key count; it only chooses the launch shape.
        mk = int(max_seqlen_k) if max_seqlen_k is not None else 0
        call = (torch.ops.fastkernels_amd.varlen_prefill if torch.compiler.is_compiling()
                else ops.varlen_prefill)
        call(out, q, k, v, cu_seqlens_q, cu_seqlens_k, int(max_seqlen_q), float(softmax_scale),
             bool(causal), -1, None, mk)
        return out
