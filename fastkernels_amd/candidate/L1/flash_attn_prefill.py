"""Candidate ``FlashAttnPrefill`` for fastkernels/tasks/baseline/L1/flash_attn_prefill.py:18-74.

Same constructor ``(num_heads, num_kv_heads, head_dim)`` (with ``sm_scale``) and
``forward(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, **kwargs)``.

- With ``block_table`` (the paged path of Attention._forward_pure / _forward_mixed,
  attention_impl.py:409-434, 682-707): ``k`` / ``v`` are the NHD caches
  ``[num_blocks, block_size, Hk, D]`` and sequence b's keys are its first
  ``cu_seqlens_k[b+1] - cu_seqlens_k[b]`` cached tokens (the reference's ``seqused_k``).
- Without it: ``k`` / ``v`` are ``[total_k, Hk, D]`` and sequence b's keys are rows
  ``cu_seqlens_k[b] .. cu_seqlens_k[b+1]``.

Keyword arguments: ``softmax_scale`` (default ``head_dim ** -0.5``), ``causal``
(default True; queries aligned to the end of the keys), ``out``, fp8 descales
``k_descale`` / ``v_descale`` (or ``k_scale`` / ``v_scale``) for float8_e4m3fn
caches, ``window_size`` (causal sliding window ``(left, right)``: query j keeps
its last left + 1 positions; left = -1 is no window; a window with
``causal=False`` raises NotImplementedError) and ``s_aux`` (attention-sink
logits, one per query head) as ``Attention._forward_pure`` passes them
(attention_impl.py:401-434).  ``max_seqlen_q`` must bound every query chunk (it
sizes the launch); no host synchronisation happens.  Returns
``[total_q, num_heads, head_dim]``.

Head sizes (``ops.PREFILL_HEADS``): 32, 64, 72, 80, 96, 128 and 256 with bf16 keys
(72 and 80 are Qwen3-VL's and Qwen2/2.5-VL's vision encoders, L2/vision_attention.py:
32,39), 64, 128 and 256 with fp8 pages; the constructor refuses others.
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


class FlashAttnPrefill(nn.Module):
    def __init__(self, num_heads: int, num_kv_heads: int, head_dim: int):
        super().__init__()
        if not ops.prefill_heads_supported(head_dim):
            # Refused here rather than at the first forward.
            raise NotImplementedError(
                f"FlashAttnPrefill (gfx950): head_dim {head_dim} is not built (bf16: "
                f"{sorted(d for d, dv in ops.PREFILL_HEADS if d == dv)}; fp8 pages: 64, 128, 256)")
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.sm_scale = head_dim ** -0.5
        self._sinks_src = None  # (tensor, version) of the cached float32 s_aux copy
        self._sinks_f32: torch.Tensor | None = None

    def _sinks(self, s_aux, device) -> torch.Tensor | None:
        """s_aux as contiguous float32 [num_heads] on the device, converted once per
        source tensor version (the layer passes the same sinks parameter each step)."""
        if s_aux is None:
            return None
        if not isinstance(s_aux, torch.Tensor) or s_aux.numel() != self.num_heads:
            raise ValueError(f"FlashAttnPrefill: s_aux must hold {self.num_heads} logits")
        if s_aux.dtype == torch.float32 and s_aux.is_contiguous() and s_aux.device == device:
            return s_aux.reshape(-1)
        src = self._sinks_src
        if (self._sinks_f32 is None or src is None or src[0] is not s_aux
                or src[1] != s_aux._version or self._sinks_f32.device != device):
            if device.type == "cuda" and torch.cuda.is_current_stream_capturing():
                raise RuntimeError("FlashAttnPrefill: convert s_aux to float32 before graph "
                                   "capture (run the step eagerly once)")
            self._sinks_f32 = s_aux.detach().to(device=device, dtype=torch.float32).reshape(-1)
            self._sinks_src = (s_aux, s_aux._version)
        return self._sinks_f32

    @staticmethod
    def _scale_vec(s, hk: int, device) -> torch.Tensor | None:
        if s is None:
            return None
        if not isinstance(s, torch.Tensor):
            s = torch.tensor([float(s)], dtype=torch.float32)
        s = s.to(device=device, dtype=torch.float32).reshape(-1)
        if s.numel() == 1:
            s = s.expand(hk)
        if s.numel() != hk:
            raise ValueError(f"FlashAttnPrefill: fp8 scale must have 1 or {hk} entries")
        return s.contiguous()

    def forward(self, q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                **kwargs):
        block_table = kwargs.pop("block_table", None)
        softmax_scale = kwargs.pop("softmax_scale", None)
        causal = bool(kwargs.pop("causal", True))
        out = kwargs.pop("out", None)
        k_scale = kwargs.pop("k_scale", kwargs.pop("k_descale", None))
        v_scale = kwargs.pop("v_scale", kwargs.pop("v_descale", None))
        window = kwargs.pop("window_size", (-1, -1))
        s_aux = kwargs.pop("s_aux", None)
        for ignored in ("scheduler_metadata", "num_splits", "seqused_k", "fa_version"):
            kwargs.pop(ignored, None)
        if kwargs:
            raise TypeError(f"FlashAttnPrefill: unexpected arguments {sorted(kwargs)}")
        window_left = -1
        if window is not None and tuple(window) != (-1, -1):
            if not causal:
                raise NotImplementedError("FlashAttnPrefill (gfx950): a sliding window needs "
                                          "causal=True")
            window_left = int(window[0]) if int(window[0]) >= 0 else -1
        sinks = self._sinks(s_aux, q.device)
        if softmax_scale is None:
            softmax_scale = self.sm_scale
        # A bound on every sequence's key count; it only chooses the launch shape.
        mk = int(max_seqlen_k) if max_seqlen_k is not None else 0
        total = q.shape[0]
        q3 = q.view(total, self.num_heads, self.head_dim)
        if cu_seqlens_q.dtype != torch.int32:
            cu_seqlens_q = cu_seqlens_q.to(torch.int32)
        if cu_seqlens_k.dtype != torch.int32:
            cu_seqlens_k = cu_seqlens_k.to(torch.int32)
        if out is None:
            out = torch.empty((total, self.num_heads, self.head_dim), dtype=q.dtype,
                              device=q.device)
        out3 = out.view(total, self.num_heads, self.head_dim)
        compiling = torch.compiler.is_compiling()
        if block_table is not None:
            if block_table.dtype != torch.int32:
                block_table = block_table.to(torch.int32)
            hk = k.shape[2]
            ks = self._scale_vec(k_scale, hk, q.device)
            vs = self._scale_vec(v_scale, hk, q.device)
            call = torch.ops.fastkernels_amd.paged_prefill if compiling else ops.paged_prefill
            call(out3, q3, k, v, block_table, cu_seqlens_q, cu_seqlens_k, int(max_seqlen_q),
                 float(softmax_scale), ks, vs, causal, window_left, sinks, mk)
        else:
            hk = k.shape[-2] if k.dim() == 3 else k.shape[-1] // self.head_dim
            k3 = k.view(k.shape[0], hk, self.head_dim)
            v3 = v.view(v.shape[0], hk, self.head_dim)
            call = torch.ops.fastkernels_amd.varlen_prefill if compiling else ops.varlen_prefill
            call(out3, q3, k3, v3, cu_seqlens_q, cu_seqlens_k, int(max_seqlen_q),
                 float(softmax_scale), causal, window_left, sinks, mk)
        return out
