"""The reference's PyTorch paths of the decode-step ops, restated for the CPU
baseline legs.

TEST INFRASTRUCTURE ONLY (like the rest of ``oracle/``): ``bench.py``'s
``cpu_baseline`` leg and its per-op table time these on the host's cores, and
``tests/`` pin them against the numpy oracle.  Nothing in ``fastkernels_amd``
imports them.

- ``rms_norm_native``: ``RMSNorm.forward_native`` (L1/rms_norm.py:97-118).
- ``rotary_native``: ``RotaryEmbedding.forward_native``, NeoX pairing
  (L1/rotary_emb.py:110-139).
- ``store_kvcache_torch``: the store as a torch scatter into the flattened caches
  (what ``_store_kvcache_kernel``, L1/store_kvcache.py:16-35, does per token;
  the reference has no CPU path).
- ``silu_and_mul_native``: ``SiluAndMul.forward_native`` (L1/silu_and_mul.py:19-22).

``decode_torch`` follows ``Attention._decode_torch`` and its helpers
(fastkernels/tasks/baseline/L2/attention_impl.py:592-664) op for op, on CPU
tensors in the caller's dtype (bf16 for C3):

- ``_cache_seq`` (:598-604): ``cache[block_table[:pages].long()]`` reshaped to
  ``[-1, Hk, D]`` and cut to the sequence length;
- ``_repeat_kv_for_heads`` (:592-596): ``repeat_interleave(Hq / Hk, dim=1)``;
- ``_sdpa_one`` (:606-622): SDPA over ``[1, H, len, D]`` views with the boolean
  mask ``k_pos <= key_offset + q_pos``, ``key_offset = len - 1`` for a decode
  query (every cached key visible), ``scale`` = the layer's softmax scale.

fp8 pages are dequantised after the gather as ``_cast_kv_tile`` does
(triton_unified_attention.py:64-67): ``(float(x) * scale).to(q.dtype)``, with
one scale per kv head.
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


def _dequant(seq: torch.Tensor, scale, dtype) -> torch.Tensor:
    if seq.dtype != torch.float8_e4m3fn:
        return seq
    s = torch.ones(1, seq.shape[1], 1) if scale is None else scale.float().reshape(1, -1, 1)
    return (seq.float() * s).to(dtype)


def decode_torch(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                 cache_seqlens: torch.Tensor, block_tables: torch.Tensor, scale: float,
                 seqs=None, k_scale=None, v_scale=None) -> torch.Tensor:
    """Decode attention [B, Hq, D] in q's dtype: one SDPA per sequence over its gathered
    pages.  ``seqs`` restricts the sequences computed (the others stay 0); fp8 caches
    take per-kv-head ``k_scale`` / ``v_scale`` (None: 1)."""
    out = torch.zeros_like(q)
    for i in (range(q.shape[0]) if seqs is None else seqs):
        n = int(cache_seqlens[i])
        k_seq = _dequant(_cache_seq(k_cache, block_tables[i], n), k_scale, q.dtype)
        v_seq = _dequant(_cache_seq(v_cache, block_tables[i], n), v_scale, q.dtype)
        out[i:i + 1] = _sdpa_one(q[i:i + 1], k_seq, v_seq, scale, key_offset=n - 1)
    return out


def rms_norm_native(x: torch.Tensor, weight: torch.Tensor | None, eps: float,
                    residual: torch.Tensor | None = None):
    """out = (x32 * rsqrt(mean(x32^2) + eps)).to(dtype) * weight, with x32 = x (+ residual)
    in fp32 and the new residual = x32 rounded to x's dtype; returns out or (out, residual)."""
    dtype = x.dtype
    xf = x.float()
    if residual is not None:
        xf = xf + residual.float()
        residual = xf.to(dtype)
    xf = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    out = xf.to(dtype)
    if weight is not None:
        out = out * weight
    return out if residual is None else (out, residual)


def rotary_native(positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor,
                  head_dim: int, cos_sin_cache: torch.Tensor):
    """NeoX rotation of q [T, Hq*D] and k [T, Hk*D] by cache rows [cos | sin]: for
    i < D/2, o[i] = x[i] cos - x[i + D/2] sin, o[i + D/2] = x[i + D/2] cos + x[i] sin."""
    cs = cos_sin_cache[positions]
    half = cs.shape[-1] // 2
    cos, sin = cs[..., :half].unsqueeze(1), cs[..., half:].unsqueeze(1)

    def rot(x):
        x = x.view(x.shape[0], -1, head_dim)
        a, b = x[..., :half], x[..., half:]
        return torch.cat([a * cos - b * sin, b * cos + a * sin], dim=-1).flatten(1)

    return rot(query), rot(key)


def store_kvcache_torch(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                        v_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """Row i of key / value [N, Hk, D] into cache slot slot_mapping[i] (negative:
    skipped) of the flattened [slots, Hk * D] caches, in place."""
    keep = slot_mapping >= 0
    slots = slot_mapping[keep].to(torch.long)
    kf = k_cache.view(-1, key.shape[1] * key.shape[2])
    vf = v_cache.view(-1, value.shape[1] * value.shape[2])
    kf.index_copy_(0, slots, key[keep].reshape(slots.numel(), -1))
    vf.index_copy_(0, slots, value[keep].reshape(slots.numel(), -1))


def silu_and_mul_native(x: torch.Tensor) -> torch.Tensor:
    """silu(x[..., :d]) * x[..., d:] with d = x.shape[-1] / 2."""
    d = x.shape[-1] // 2
    return F.silu(x[..., :d]) * x[..., d:]
