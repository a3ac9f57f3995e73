"""Candidate ``FlashAttnVarlen`` for fastkernels/tasks/baseline/L1/flash_attn_varlen.py:21-47.

Variable-length attention over dense (no block table) query / key / value tensors:
``forward(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
softmax_scale, causal=True, return_softmax_lse=False)`` with ``q [total_q, Hq, D]``,
``k [total_k, Hk, D]`` and ``v [total_k, Hk, Dv]`` (rows ``cu_seqlens_k[b] ..
cu_seqlens_k[b+1]`` are sequence b's keys; ``Hq`` a multiple of ``Hk``); causal
queries are aligned to the end of their sequence's keys, as in
flash_attn_varlen_func.  Returns ``[total_q, Hq, Dv]`` in q's dtype, and with
``return_softmax_lse=True`` the pair ``(out, lse)``, lse float32 ``[Hq, total_q]``
holding ln(sum over visible keys of e^(softmax_scale q.k)) per row (-inf for a row
with no visible key; flash-attn's own binary writes +inf there, which
``merge_attn_states`` reads the same way).

The reference's callers: the encoder attention (L2/encoder_attention.py:37,
bidirectional) and MLA prefill (L2/mla_attention_impl.py:347-398: causal over the
new tokens, and non-causal over each cached-context chunk with the LSE, merged by
``merge_attn_states``; query / key head 192, value head 128).

It runs on the gfx950 kernel of ``FlashAttnPrefill``'s dense path
(``fk_varlen_prefill``), bf16, at the head sizes ``ops.PREFILL_HEADS`` lists
(equal sizes 32, 64, 72, 80, 96, 128, 256, and 192 / 128).  Other sizes raise
``NotImplementedError`` (the class takes no head size at construction, so this is
the first point where it can tell).
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
        if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
            raise ValueError("FlashAttnVarlen: q, k, v must be [tokens, heads, head_dim]")
        total, hq, d = q.shape
        dv = v.shape[2]
        if k.shape[2] != d:
            raise ValueError(f"FlashAttnVarlen: query and key head sizes differ ({d}, "
                             f"{k.shape[2]})")
        if not ops.prefill_heads_supported(d, dv):
            raise NotImplementedError(f"FlashAttnVarlen (gfx950): head sizes {d} / {dv} are not "
                                      f"built (query / key, value: {sorted(ops.PREFILL_HEADS)})")
        if cu_seqlens_q.dtype != torch.int32:
            cu_seqlens_q = cu_seqlens_q.to(torch.int32)
        if cu_seqlens_k.dtype != torch.int32:
            cu_seqlens_k = cu_seqlens_k.to(torch.int32)
        out = torch.empty((total, hq, dv), dtype=q.dtype, device=q.device)
        lse = (torch.empty((hq, total), dtype=torch.float32, device=q.device)
               if return_softmax_lse else None)
        # A bound on every sequence's key count; it only chooses the launch shape.
        mk = int(max_seqlen_k) if max_seqlen_k is not None else 0
        call = (torch.ops.fastkernels_amd.varlen_prefill if torch.compiler.is_compiling()
                else ops.varlen_prefill)
        call(out, q, k, v, cu_seqlens_q, cu_seqlens_k, int(max_seqlen_q), float(softmax_scale),
             bool(causal), -1, None, mk, lse)
        return (out, lse) if return_softmax_lse else out
