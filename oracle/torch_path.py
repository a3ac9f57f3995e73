"""The reference's PyTorch decode path, restated for the CPU baseline leg.

TEST INFRASTRUCTURE ONLY (like the rest of ``oracle/``): ``bench.py``'s
``cpu_baseline`` leg times it on the host's cores, and ``tests/`` pin it against
the numpy oracle.  Nothing in ``fastkernels_amd`` imports it.

``decode_torch`` follows ``Attention._decode_torch`` and its helpers
(fastkernels/tasks/baseline/L2/attention_impl.py:592-664) op for op, on CPU
tensors in the caller's dtype (bf16 for C3):

- ``_cache_seq`` (:598-604): ``cache[block_table[:pages].long()]`` reshaped to
  ``[-1, Hk, D]`` and cut to the sequence length;
- ``_repeat_kv_for_heads`` (:592-596): ``repeat_interleave(Hq / Hk, dim=1)``;
- ``_sdpa_one`` (:606-622): SDPA over ``[1, H, len, D]`` views with the boolean
  mask ``k_pos <= key_offset + q_pos``, ``key_offset = len - 1`` for a decode
  query (every cached key visible), ``scale`` = the layer's softmax scale.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def _cache_seq(cache: torch.Tensor, block_row: torch.Tensor, length: int) -> torch.Tensor:
    bs, hk, d = cache.shape[1:]
    pages = (length + bs - 1) // bs
    ids = block_row[:pages].to(torch.long)
    return cache[ids].reshape(-1, hk, d)[:length]


def _sdpa_one(q_seq: torch.Tensor, k_seq: torch.Tensor, v_seq: torch.Tensor, scale: float,
              key_offset: int) -> torch.Tensor:
    hq, hk = q_seq.shape[1], k_seq.shape[1]
    if hq != hk:
        k_seq = k_seq.repeat_interleave(hq // hk, dim=1)
        v_seq = v_seq.repeat_interleave(hq // hk, dim=1)
    q4 = q_seq.transpose(0, 1).unsqueeze(0)
    k4 = k_seq.transpose(0, 1).unsqueeze(0)
    v4 = v_seq.transpose(0, 1).unsqueeze(0)
    q_pos = key_offset + torch.arange(q_seq.shape[0])
    k_pos = torch.arange(k_seq.shape[0])
    mask = k_pos.unsqueeze(0) <= q_pos.unsqueeze(1)
    out = F.scaled_dot_product_attention(q4, k4, v4, attn_mask=mask, dropout_p=0.0, scale=scale)
    return out.squeeze(0).transpose(0, 1)


def decode_torch(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                 cache_seqlens: torch.Tensor, block_tables: torch.Tensor, scale: float,
                 seqs=None) -> torch.Tensor:
    """Decode attention [B, Hq, D] in q's dtype: one SDPA per sequence over its gathered
    pages.  ``seqs`` restricts the sequences computed (the others stay 0)."""
    out = torch.zeros_like(q)
    for i in (range(q.shape[0]) if seqs is None else seqs):
        n = int(cache_seqlens[i])
        k_seq = _cache_seq(k_cache, block_tables[i], n)
        v_seq = _cache_seq(v_cache, block_tables[i], n)
        out[i:i + 1] = _sdpa_one(q[i:i + 1], k_seq, v_seq, scale, key_offset=n - 1)
    return out
