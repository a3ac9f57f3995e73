"""Candidate ``FlashAttnDecode`` for fastkernels/tasks/baseline/L1/flash_attn_decode.py:22-181.

Same constructor ``(num_heads, num_kv_heads, head_dim, page_size=None)`` and
``forward(q, k_cache, v_cache, cache_seqlens=None, **kwargs)`` with the kwargs
the reference forwards to ``flash_attn_varlen_func`` (flash_attn_decode.py:
113-181): ``block_table``, ``max_seq_len``, ``softmax_scale``, ``causal``
(decode: every cached key is visible), ``num_splits``, ``out``,
``window_size`` (default: the ``_window_size`` attribute that
``Attention.__init__`` sets, attention_impl.py:242-244, :282; ``(left, right)``
with left >= 0 keeps the last left + 1 keys) and ``s_aux`` (attention-sink
logits, one per query head, attention_impl.py:401-406).  Returns
``[B, num_heads, head_dim]`` in q's dtype.

The engine's FA3 hooks work unchanged: ``preallocate(max_batch_size, device)``
(engine.py:1545), the shared ``_cu_seqlens_q`` / ``_sched_buf`` / ``_sched_meta``
attributes it copies between grouped ops, ``_force_graph_splits``, and
``update_scheduler_metadata``.  ``fa_version`` is None, so the engine's
scheduler refresh (fa_utils.py:120-145) skips this op: its schedule is computed
on the device from the lengths of each call.

The gfx950 kernel is split-context flash-decoding.  By default
(``num_splits`` 0) the 16-token tiles of all sequences are cut into equal
ranges, one work-group per CU, so mixed lengths leave no idle tail; an explicit
``num_splits`` uses that many fixed partitions per sequence instead.  Sequences
cut across work-groups leave partials in a per-module workspace that a second
kernel merges with the log-sum-exp rule.
The workspace is allocated outside graph capture (like the reference's
persistent FA3 scheduler buffer, flash_attn_decode.py:87-111) and only grows;
inside a capture it must already be large enough.

fp8 KV: caches of dtype ``torch.float8_e4m3fn`` are dequantised per kv head
with ``k_scale`` / ``v_scale`` (float32 [num_kv_heads]; per-tensor scales may be
given as a single value and are broadcast), i.e. K = float(K8) * k_scale as in
``_cast_kv_tile`` (triton_unified_attention.py:51-67).  FA-style
``k_descale`` / ``v_descale`` are accepted as aliases.

``forward_store(q, key, value, k_cache, v_cache, slot_mapping, cache_seqlens,
**kwargs)`` is the decode step of ``Attention.forward_impl`` (store, then decode)
in one launch.

No host synchronisation: the default length-balanced schedule reads the context
lengths on the device, and when ``max_seq_len`` is absent the bound used for
fixed partitions is the block table width (``block_table.shape[1] * page_size``)
instead of ``cache_seqlens.max().item()`` (flash_attn_decode.py:122-125).
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


# Head sizes the decode kernel is built for (Whisper 64; Llama / Qwen3 128;
# Qwen3-Next, Gemma 256).
DECODE_HEAD_SIZES = (64, 128, 256)


class FlashAttnDecode(nn.Module):
    def __init__(self, num_heads: int, num_kv_heads: int, head_dim: int,
                 page_size: int | None = None):
        super().__init__()
        if head_dim not in DECODE_HEAD_SIZES:
            # Refused here rather than at the first forward.
            raise NotImplementedError(f"FlashAttnDecode (gfx950): head_dim {head_dim} is not "
                                      f"built (head sizes {DECODE_HEAD_SIZES})")
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.page_size = page_size
        self._workspace: torch.Tensor | None = None
        # Attributes the reference's engine reads or shares between grouped decode
        # ops (engine.py:1538-1550, fa_utils.py:108-145, jamba_engine.py:719-856).
        self.fa_version = None
        self._cu_seqlens_q: torch.Tensor | None = None
        self._sched_buf: torch.Tensor | None = None
        self._sched_meta: torch.Tensor | None = None
        self._graph_num_splits = 32
        self._force_graph_splits = False
        self._window_size = (-1, -1)
        self._qkv_dtype = torch.bfloat16
        self._sinks_src = None  # (tensor, version) of the cached float32 s_aux copy
        self._sinks_f32: torch.Tensor | None = None

    def _get_workspace(self, nbytes: int, device: torch.device) -> torch.Tensor | None:
        if nbytes <= 0:
            return None
        ws = self._workspace
        if ws is None or ws.device != device or ws.numel() < nbytes:
            if device.type == "cuda" and torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    "FlashAttnDecode: split-context workspace must be allocated before graph "
                    f"capture ({nbytes} bytes needed); call preallocate() or run eagerly once")
            ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
            self._workspace = ws
        return ws

    def preallocate(self, max_batch_size: int, device: torch.device,
                    max_seq_len: int | None = None, num_splits: int = 0) -> None:
        """Allocate graph-stable buffers for batches up to max_batch_size, outside
        capture: the reference's signature (flash_attn_decode.py:97-111, called at
        engine.py:1545).  The default (length-balanced) schedule's workspace does not
        depend on the context lengths; a fixed ``num_splits`` also needs the
        ``max_seq_len`` bound."""
        device = torch.device(device)
        if self._cu_seqlens_q is None or self._cu_seqlens_q.numel() < max_batch_size + 1:
            self._cu_seqlens_q = torch.arange(max_batch_size + 1, dtype=torch.int32,
                                              device=device)
        if num_splits and max_seq_len is None:
            raise ValueError("FlashAttnDecode.preallocate: num_splits needs max_seq_len")
        plan = ops.paged_decode_plan(max_batch_size, self.num_heads, self.num_kv_heads,
                                     self.head_dim, int(max_seq_len or 1), num_splits)
        self._get_workspace(plan.workspace_bytes, device)

    def update_scheduler_metadata(self, cache_seqlens: torch.Tensor, max_seqlen_k: int,
                                  qkv_dtype: torch.dtype | None = None,
                                  window_size: tuple[int, int] = (-1, -1),
                                  max_seqlen_q: int = 1) -> None:
        """The reference recomputes FA3 tile-scheduler metadata here
        (flash_attn_decode.py:50-95).  The gfx950 kernel reads the lengths on the
        device at every call, so only the window and dtype are recorded."""
        if qkv_dtype is not None:
            self._qkv_dtype = qkv_dtype
        self._window_size = tuple(window_size)
        self._sched_meta = None

    def _sinks(self, s_aux, device) -> torch.Tensor | None:
        """s_aux as contiguous float32 [num_heads] on the device; the copy is kept
        while the source tensor is unchanged (the layer passes the same sinks
        parameter every step), so a decode step makes no conversion."""
        if s_aux is None:
            return None
        if not isinstance(s_aux, torch.Tensor):
            raise TypeError("FlashAttnDecode: s_aux must be a tensor of num_heads logits")
        if s_aux.numel() != self.num_heads:
            raise ValueError(f"FlashAttnDecode: s_aux must have {self.num_heads} entries")
        if s_aux.dtype == torch.float32 and s_aux.is_contiguous() and s_aux.device == device:
            return s_aux.reshape(-1)
        if device.type != "cuda":
            return s_aux.detach().to(device=device, dtype=torch.float32).reshape(-1)
        key = (s_aux, s_aux._version)
        src = self._sinks_src
        if self._sinks_f32 is None or src is None or src[0] is not s_aux or src[1] != key[1] \
                or self._sinks_f32.device != device:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("FlashAttnDecode: convert s_aux to float32 before graph "
                                   "capture (run the step eagerly once)")
            self._sinks_f32 = s_aux.detach().to(device=device, dtype=torch.float32).reshape(-1)
            self._sinks_src = key
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
            raise ValueError(f"FlashAttnDecode: fp8 scale must have 1 or {hk} entries")
        return s.contiguous()

    def _launch_args(self, q, k_cache, cache_seqlens, kwargs):
        """Parses the reference's decode kwargs; returns what both launch paths need."""
        max_seq_len = kwargs.pop("max_seq_len", None)
        block_table = kwargs.pop("block_table", None)
        softmax_scale = kwargs.pop("softmax_scale", None)
        kwargs.pop("causal", None)
        num_splits = int(kwargs.pop("num_splits", 0) or 0)
        out = kwargs.pop("out", None)
        k_scale = kwargs.pop("k_scale", kwargs.pop("k_descale", None))
        v_scale = kwargs.pop("v_scale", kwargs.pop("v_descale", None))
        window = kwargs.pop("window_size", None)
        if window is None:
            window = self._window_size
        s_aux = kwargs.pop("s_aux", None)
        kwargs.pop("scheduler_metadata", None)
        # A decode query is the last token, so only the left extent matters.
        window_left = int(window[0]) if window is not None and int(window[0]) >= 0 else -1
        if kwargs:
            raise TypeError(f"FlashAttnDecode: unexpected arguments {sorted(kwargs)}")
        sinks = self._sinks(s_aux, q.device)
        if block_table is None or cache_seqlens is None:
            raise ValueError("FlashAttnDecode: block_table and cache_seqlens are required")

        b = q.shape[0]
        block_size = k_cache.shape[1]
        if block_table.dtype != torch.int32:
            block_table = block_table.to(torch.int32)
        if cache_seqlens.dtype != torch.int32:
            cache_seqlens = cache_seqlens.to(torch.int32)
        if max_seq_len is None:
            max_seq_len = block_table.shape[1] * block_size
        if softmax_scale is None:
            softmax_scale = ops.default_softmax_scale(self.head_dim)
        hk = k_cache.shape[2]
        k_scale = self._scale_vec(k_scale, hk, q.device)
        v_scale = self._scale_vec(v_scale, hk, q.device)

        plan = ops.paged_decode_plan(b, self.num_heads, hk, self.head_dim, int(max_seq_len),
                                     num_splits)
        ws = self._get_workspace(plan.workspace_bytes, q.device)
        if out is None:
            out = torch.empty((b, self.num_heads, self.head_dim), dtype=q.dtype, device=q.device)
        return dict(out=out, block_table=block_table, cache_seqlens=cache_seqlens,
                    softmax_scale=float(softmax_scale), part_tokens=plan.part_tokens,
                    max_parts=plan.max_parts, ws=ws, k_scale=k_scale, v_scale=v_scale,
                    window_left=window_left, sinks=sinks)

    def forward(self, q, k_cache, v_cache, cache_seqlens=None, **kwargs):
        a = self._launch_args(q, k_cache, cache_seqlens, kwargs)
        b = q.shape[0]
        q3 = q.view(b, self.num_heads, self.head_dim)
        out3 = a["out"].view(b, self.num_heads, self.head_dim)
        call = torch.ops.fastkernels_amd.paged_decode if torch.compiler.is_compiling() \
            else ops.paged_decode
        call(out3, q3, k_cache, v_cache, a["block_table"], a["cache_seqlens"], a["softmax_scale"],
             a["part_tokens"], a["max_parts"], a["ws"], a["k_scale"], a["v_scale"],
             a["window_left"], a["sinks"])
        return a["out"]

    def forward_store(self, q, key, value, k_cache, v_cache, slot_mapping, cache_seqlens=None,
                      **kwargs):
        """``StoreKVCache()(key, value, k_cache, v_cache, slot_mapping)`` then
        ``forward(q, k_cache, v_cache, cache_seqlens, **kwargs)`` in one launch: the
        decode step of Attention.forward_impl (attention_impl.py:313-363, :436-450).

        Token b must be sequence b's new token: slot_mapping[b] is -1 or the slot of
        position cache_seqlens[b] - 1 in block_table[b], as the engine's decode step
        builds it (engine.py:5020-5024).  The cache and the output then equal the
        two separate calls bit for bit."""
        a = self._launch_args(q, k_cache, cache_seqlens, kwargs)
        b = q.shape[0]
        hk = k_cache.shape[2]
        q3 = q.view(b, self.num_heads, self.head_dim)
        k3 = key.view(b, hk, self.head_dim)
        v3 = value.view(b, hk, self.head_dim)
        if key.dtype != k_cache.dtype:
            # A converting store (e.g. bf16 rows into an fp8 cache) is a launch of its
            # own; the decode then reads the cache as usual.
            ops.store_kvcache(k3, v3, k_cache, v_cache, slot_mapping)
            out3 = a["out"].view(b, self.num_heads, self.head_dim)
            ops.paged_decode(out3, q3, k_cache, v_cache, a["block_table"], a["cache_seqlens"],
                             a["softmax_scale"], a["part_tokens"], a["max_parts"], a["ws"],
                             a["k_scale"], a["v_scale"], a["window_left"], a["sinks"])
            return a["out"]
        out3 = a["out"].view(b, self.num_heads, self.head_dim)
        call = torch.ops.fastkernels_amd.store_paged_decode if torch.compiler.is_compiling() \
            else ops.store_paged_decode
        call(out3, q3, k3, v3, k_cache, v_cache, slot_mapping, a["block_table"],
             a["cache_seqlens"], a["softmax_scale"], a["part_tokens"], a["max_parts"], a["ws"],
             a["k_scale"], a["v_scale"], a["window_left"], a["sinks"])
        return a["out"]
