"""Candidates ``RotaryEmbedding`` and ``Gemma4ProportionalRotaryEmbedding`` for
fastkernels/tasks/baseline/L1/rotary_emb.py:71-230.

Same constructor (including the Llama-3.1 frequency scaling of
rotary_emb.py:44-68,95-102), the same ``cos_sin_cache`` buffer
([max_position, rot_dim] float32, cos then sin, rotary_emb.py:104-107), and
``forward(positions, query, key)`` rotating query/key in place and returning
them (rotary_emb.py:179-191).  ``forward_store(positions, query, key, value,
k_cache, v_cache, slot_mapping, q_norm=None, k_norm=None)`` additionally applies
Qwen3's per-head q/k RMSNorm first and stores the rotated key and the value
rows in the paged cache, in one launch.  The kernel reads the float32 cache directly and
rounds cos/sin to the query dtype itself, so no per-call cache cast is made
(the reference casts the whole cache on every call when it is float32,
rotary_emb.py:171-173).
"""
from __future__ import annotations

import math
import sys
from pathlib import Path

import torch
import torch.nn as nn

try:
    import fastkernels_amd  # noqa: F401
except ImportError:  # loaded by file path from the reference harness
    sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
from fastkernels_amd import ops


def _llama31_inv_freq(inv_freq: torch.Tensor, factor: float, low_freq_factor: float,
                      high_freq_factor: float, original_max_pos: int) -> torch.Tensor:
    """Llama-3.1 piecewise frequency scaling (rotary_emb.py:44-68)."""
    wavelen = 2 * math.pi / inv_freq
    low_wavelen = original_max_pos / low_freq_factor
    high_wavelen = original_max_pos / high_freq_factor
    if low_freq_factor != high_freq_factor:
        smooth = (original_max_pos / wavelen - low_freq_factor) / (high_freq_factor - low_freq_factor)
    else:
        smooth = torch.zeros_like(inv_freq)
    blended = (1 - smooth) * inv_freq / factor + smooth * inv_freq
    scaled = torch.where(wavelen > low_wavelen, inv_freq / factor, blended)
    return torch.where(wavelen < high_wavelen, inv_freq, scaled)


class RotaryEmbedding(nn.Module):
    def __init__(self, head_dim: int, max_position_embeddings: int, rope_theta: float,
                 rope_scaling_factor: float = 1.0, rope_low_freq_factor: float = 1.0,
                 rope_high_freq_factor: float = 1.0,
                 rope_original_max_position_embeddings: int | None = None,
                 is_neox_style: bool = True):
        super().__init__()
        self.head_dim = head_dim
        self.is_neox_style = is_neox_style
        exponents = torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim
        inv_freq = 1.0 / (rope_theta ** exponents)
        if rope_scaling_factor != 1.0 and rope_original_max_position_embeddings is not None:
            inv_freq = _llama31_inv_freq(inv_freq, rope_scaling_factor, rope_low_freq_factor,
                                         rope_high_freq_factor,
                                         rope_original_max_position_embeddings)
        angles = torch.outer(torch.arange(max_position_embeddings, dtype=torch.float), inv_freq)
        cache = torch.cat((angles.cos(), angles.sin()), dim=-1).float()
        self.register_buffer("cos_sin_cache", cache, persistent=False)

    def _cache_for(self, query: torch.Tensor) -> torch.Tensor:
        cache = self.cos_sin_cache
        if cache.device != query.device:
            cache = cache.to(query.device)
        if cache.dtype not in (torch.float32, query.dtype):
            cache = cache.to(query.dtype)
        return cache

    def forward_store(self, positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor,
                      value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                      slot_mapping: torch.Tensor, q_norm: nn.Module | None = None,
                      k_norm: nn.Module | None = None):
        """The attention block's q/k path in one launch: ``q_norm`` / ``k_norm``
        per head (Qwen3, attention.py:120-135; RMSNorm modules or None), this
        rotation (:137-139), then ``StoreKVCache()(key, value, k_cache, v_cache,
        slot_mapping)`` (attention_impl.py:323-325).  query / key ([T, H*D] views,
        e.g. slices of the fused qkv output) are rewritten in place and returned."""
        if (q_norm is None) != (k_norm is None):
            raise ValueError("RotaryEmbedding.forward_store: pass both q_norm and k_norm, or neither")
        qw = kw = None
        eps = 1e-6
        if q_norm is not None:
            if q_norm.eps != k_norm.eps:
                raise ValueError("RotaryEmbedding.forward_store: q_norm and k_norm eps differ")
            eps = q_norm.eps
            qw = (q_norm.weight if q_norm.elementwise_affine else q_norm._unit_weight).detach()
            kw = (k_norm.weight if k_norm.elementwise_affine else k_norm._unit_weight).detach()
            qw = qw.to(device=query.device, dtype=query.dtype).contiguous()
            kw = kw.to(device=query.device, dtype=query.dtype).contiguous()
        cache = self._cache_for(query)
        if positions.dtype != torch.int64:
            positions = positions.to(torch.int64)
        if not positions.is_contiguous():
            positions = positions.contiguous()
        k3 = k_cache.view(k_cache.shape[0], k_cache.shape[1], -1, self.head_dim)
        v3 = v_cache.view(v_cache.shape[0], v_cache.shape[1], -1, self.head_dim)
        if k_cache.dtype != query.dtype:
            # A cache of another dtype (fp8): the fused kernel stores bit copies, so
            # run the ops one by one, the store converting as tl.store does.
            t = positions.numel()
            if q_norm is not None:
                query.view(t, -1, self.head_dim).copy_(q_norm(query.view(t, -1, self.head_dim)))
                key.view(t, -1, self.head_dim).copy_(k_norm(key.view(t, -1, self.head_dim)))
            ops.rotary_embedding(positions, query, key, self.head_dim, cache, self.is_neox_style)
            hk = k3.shape[2]
            ops.store_kvcache(key.view(t, hk, self.head_dim), value.view(t, hk, self.head_dim),
                              k3, v3, slot_mapping)
            return query, key
        call = torch.ops.fastkernels_amd.qk_norm_rope_store if torch.compiler.is_compiling() \
            else ops.qk_norm_rope_store
        call(positions, query, key, value, k3, v3, slot_mapping, self.head_dim, cache,
             self.is_neox_style, qw, kw, float(eps))
        return query, key

    def forward(self, positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor | None):
        cache = self.cos_sin_cache
        if cache.device != query.device:
            cache = cache.to(query.device)
        if cache.dtype not in (torch.float32, query.dtype):
            cache = cache.to(query.dtype)
        if positions.dtype != torch.int64:
            positions = positions.to(torch.int64)
        if not positions.is_contiguous():
            positions = positions.contiguous()
        if torch.compiler.is_compiling():
            torch.ops.fastkernels_amd.rotary_embedding(positions, query, key, self.head_dim, cache,
                                                       self.is_neox_style)
        else:
            ops.rotary_embedding(positions, query, key, self.head_dim, cache, self.is_neox_style)
        return query, key


class Gemma4ProportionalRotaryEmbedding(RotaryEmbedding):
    """Gemma4 proportional RoPE (rotary_emb.py:194-230): a partial rotary factor whose
    frequency exponents are divided by the full head dimension, the non-rotated angle
    pairs kept as identity rotations (inv_freq 0, so cos 1 and sin 0).  The cache spans
    the whole head, [max_position, head_dim], built by the same float32 steps as the
    reference; forward is the base class's (NeoX pairs over the whole head)."""

    def __init__(self, head_dim: int, rotary_dim: int, max_position_embeddings: int,
                 rope_theta: float):
        nn.Module.__init__(self)
        self.head_dim = head_dim
        self.is_neox_style = True
        rope_angles = rotary_dim // 2
        nope_angles = head_dim // 2 - rope_angles
        exponents = torch.arange(0, 2 * rope_angles, 2, dtype=torch.float) / head_dim
        inv_freq = 1.0 / (rope_theta ** exponents)
        if nope_angles > 0:
            inv_freq = torch.cat([inv_freq, torch.zeros(nope_angles, dtype=torch.float)])
        angles = torch.outer(torch.arange(max_position_embeddings, dtype=torch.float), inv_freq)
        cache = torch.cat((angles.cos(), angles.sin()), dim=-1).float()
        self.register_buffer("cos_sin_cache", cache, persistent=False)
