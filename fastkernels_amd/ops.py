"""Torch-facing entry points of the gfx950 decode-step kernels.

Each function validates its tensors, then calls the C ABI (``_native``) with raw
device pointers and the current HIP stream.  Nothing here computes on the host:
every op is one or two kernel launches, enqueued asynchronously.

The same functions are registered as ``torch.library`` custom ops in the
``fastkernels_amd`` namespace with in-place mutation annotations and no-op
fake (Meta) implementations, mirroring the reference's
``fastkernels_norm::*`` (fastkernels/tasks/baseline/L1/rms_norm.py:44-69) and
``fastkernels_rope::rotary_embedding`` (rotary_emb.py:24-39) schemas, so they
stay opaque under torch.compile and are capturable in HIP graphs.
"""
from __future__ import annotations

import math
from ctypes import c_void_p
from typing import NamedTuple

import torch

from . import _native

_DTYPE_TAG = {
    torch.float32: _native.FK_DTYPE_F32,
    torch.float16: _native.FK_DTYPE_F16,
    torch.bfloat16: _native.FK_DTYPE_BF16,
}
_FP8 = getattr(torch, "float8_e4m3fn", None)


def _tag(t: torch.Tensor, what: str) -> int:
    try:
        return _DTYPE_TAG[t.dtype]
    except KeyError:
        raise TypeError(f"{what}: unsupported dtype {t.dtype}") from None


def _stream(t: torch.Tensor) -> c_void_p:
    if t.device.type != "cuda":
        raise RuntimeError(f"fastkernels_amd ops run on the GPU only (got a {t.device} tensor)")
    return c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _ptr(t: torch.Tensor | None) -> c_void_p:
    return c_void_p(t.data_ptr() if t is not None else 0)


def _rows(t: torch.Tensor, width: int, what: str) -> tuple[int, int]:
    """(rows, row_stride) of a tensor viewed as [rows, width] with unit inner stride."""
    if t.dim() == 0:
        raise ValueError(f"{what}: expected at least one dimension")
    if t.numel() == 0:
        return 0, width
    if t.dim() == 1:
        if t.shape[0] != width or t.stride(0) != 1:
            raise ValueError(f"{what}: expected a contiguous row of {width}")
        return 1, width
    try:
        v = t.view(-1, t.shape[-1])
    except RuntimeError as e:
        raise ValueError(f"{what}: leading dimensions must be collapsible ({e})") from None
    if v.shape[-1] != width or v.stride(-1) != 1:
        raise ValueError(f"{what}: last dimension must be contiguous with size {width}")
    return v.shape[0], v.stride(0)


def _same_device(*ts: torch.Tensor) -> None:
    dev = ts[0].device
    for t in ts[1:]:
        if t is not None and t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------
def rms_norm(out: torch.Tensor, x: torch.Tensor, weight: torch.Tensor, eps: float) -> None:
    """out = rmsnorm(x) * weight (vLLM ``rms_norm(out, input, weight, eps)`` contract)."""
    hidden = x.shape[-1]
    _same_device(out, x, weight)
    if out.dtype != x.dtype or weight.dtype != x.dtype:
        raise TypeError("rms_norm: out, x and weight must share a dtype")
    if out.shape != x.shape or weight.shape != (hidden,) or not weight.is_contiguous():
        raise ValueError("rms_norm: shape mismatch")
    rows, xs = _rows(x, hidden, "rms_norm x")
    _, os_ = _rows(out, hidden, "rms_norm out")
    if rows == 0:
        return
    _native.call("fk_rmsnorm", _ptr(out), os_, _ptr(x), xs, _ptr(weight), rows, hidden,
                 float(eps), _tag(x, "rms_norm"), _stream(x))


def fused_add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                       eps: float) -> None:
    """In place: residual <- x + residual; x <- rmsnorm(residual) * weight."""
    hidden = x.shape[-1]
    _same_device(x, residual, weight)
    if residual.dtype != x.dtype or weight.dtype != x.dtype:
        raise TypeError("fused_add_rms_norm: x, residual and weight must share a dtype")
    if residual.shape != x.shape or weight.shape != (hidden,) or not weight.is_contiguous():
        raise ValueError("fused_add_rms_norm: shape mismatch")
    rows, xs = _rows(x, hidden, "fused_add_rms_norm x")
    _, rs = _rows(residual, hidden, "fused_add_rms_norm residual")
    if rows == 0:
        return
    _native.call("fk_fused_add_rmsnorm", _ptr(x), xs, _ptr(residual), rs, _ptr(weight), rows,
                 hidden, float(eps), _tag(x, "fused_add_rms_norm"), _stream(x))


# ---------------------------------------------------------------------------
# Rotary embedding
# ---------------------------------------------------------------------------
def rotary_embedding(positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor | None,
                     head_size: int, cos_sin_cache: torch.Tensor, is_neox: bool) -> None:
    """In-place rotary embedding of query (and key) rows at ``positions``."""
    if positions.dtype != torch.int64:
        raise TypeError("rotary_embedding: positions must be int64")
    tokens = positions.numel()
    if not positions.is_contiguous():
        raise ValueError("rotary_embedding: positions must be contiguous")
    _same_device(positions, query, cos_sin_cache, *([key] if key is not None else []))
    if cos_sin_cache.dim() != 2 or not cos_sin_cache.is_contiguous():
        raise ValueError("rotary_embedding: cos_sin_cache must be a contiguous [max_pos, rot_dim]")
    if cos_sin_cache.dtype not in (torch.float32, query.dtype):
        raise TypeError("rotary_embedding: cos_sin_cache must be float32 or the query dtype")
    if key is not None and key.dtype != query.dtype:
        raise TypeError("rotary_embedding: query and key must share a dtype")
    if tokens == 0:
        return
    qw = query.numel() // tokens
    if qw % head_size:
        raise ValueError("rotary_embedding: query width is not a multiple of head_size")
    try:
        q2 = query.view(tokens, qw)
    except RuntimeError as e:
        raise ValueError(f"rotary_embedding: query rows must be [heads*head_size] ({e})") from None
    if q2.stride(1) != 1:
        raise ValueError("rotary_embedding: query rows must be contiguous")
    num_heads = qw // head_size
    k_stride, num_kv = 0, 0
    if key is not None:
        kw = key.numel() // tokens
        if kw % head_size:
            raise ValueError("rotary_embedding: key width is not a multiple of head_size")
        try:
            k2 = key.view(tokens, kw)
        except RuntimeError as e:
            raise ValueError(f"rotary_embedding: key rows must be [heads*head_size] ({e})") from None
        if k2.stride(1) != 1:
            raise ValueError("rotary_embedding: key rows must be contiguous")
        k_stride, num_kv = k2.stride(0), kw // head_size
    _native.call("fk_rotary_embedding", _ptr(positions), _ptr(query), q2.stride(0), _ptr(key),
                 k_stride, _ptr(cos_sin_cache), _tag(cos_sin_cache, "rotary cache"),
                 cos_sin_cache.shape[0], tokens, num_heads, num_kv, head_size,
                 cos_sin_cache.shape[1], int(bool(is_neox)), _tag(query, "rotary_embedding"),
                 _stream(query))


# ---------------------------------------------------------------------------
# store_kvcache
# ---------------------------------------------------------------------------
_CONVERT_SRC = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
_CONVERT_DST = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2, torch.float8_e4m3fn: 3}

def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """Scatter key/value [N, Hk, D] rows into NHD caches at slot_mapping (-1 skips).
    Same dtype: a bit copy.  Otherwise each element is converted to the cache dtype
    (fp8 e4m3fn: round to nearest even, saturating at +-448), as tl.store does."""
    if key.dim() != 3 or value.shape != key.shape:
        raise ValueError("store_kvcache: key/value must be [N, num_kv_heads, head_dim]")
    n, hk, hd = key.shape
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape or tuple(k_cache.shape[2:]) != (hk, hd):
        raise ValueError("store_kvcache: caches must be [num_blocks, block_size, Hk, D]")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("store_kvcache: caches must be contiguous")
    convert = key.dtype != k_cache.dtype
    if value.dtype != key.dtype or v_cache.dtype != k_cache.dtype:
        raise TypeError("store_kvcache: key and value (and the two caches) must share a dtype")
    if convert and (key.dtype not in _CONVERT_SRC or k_cache.dtype not in _CONVERT_DST):
        raise TypeError(f"store_kvcache: no conversion from {key.dtype} to {k_cache.dtype}")
    for t, nm in ((key, "key"), (value, "value")):
        if t.stride(2) != 1 or (hk > 1 and t.stride(1) != hd):
            raise ValueError(f"store_kvcache: {nm} rows must be [Hk, D] contiguous")
    if slot_mapping.dtype not in (torch.int32, torch.int64) or not slot_mapping.is_contiguous():
        raise TypeError("store_kvcache: slot_mapping must be contiguous int32 or int64")
    if slot_mapping.numel() < n:
        raise ValueError("store_kvcache: slot_mapping shorter than the token count")
    _same_device(key, value, k_cache, v_cache, slot_mapping)
    if n == 0:
        return
    num_slots = k_cache.shape[0] * k_cache.shape[1]
    if convert:  # the reference's tl.store casts to the cache dtype
        _native.call("fk_store_kvcache_convert", _ptr(key), key.stride(0), _ptr(value),
                     value.stride(0), _CONVERT_SRC[key.dtype], _ptr(k_cache), _ptr(v_cache),
                     _CONVERT_DST[k_cache.dtype], _ptr(slot_mapping),
                     int(slot_mapping.dtype == torch.int64), n, hk * hd, num_slots, _stream(key))
        return
    _native.call("fk_store_kvcache", _ptr(key), key.stride(0), _ptr(value), value.stride(0),
                 _ptr(k_cache), _ptr(v_cache), _ptr(slot_mapping),
                 int(slot_mapping.dtype == torch.int64), n, hk * hd, key.element_size(),
                 num_slots, _stream(key))



def store_kvcache_hnd(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                      v_cache: torch.Tensor, slot_mapping: torch.Tensor,
                      page_size: int | None = None) -> None:
    """Scatter key/value [N, Hk, D] rows into HND caches [num_blocks, Hk, page_size, D]:
    token i's head h row goes to cache[s // page_size, h, s % page_size] with
    s = slot_mapping[i] (-1 skips), bit for bit (StoreKVCacheHND, store_kvcache.py:85-99).
    Key and cache dtypes must match (a converting HND store is not provided)."""
    if key.dim() != 3 or value.shape != key.shape:
        raise ValueError("store_kvcache_hnd: key/value must be [N, num_kv_heads, head_dim]")
    n, hk, hd = key.shape
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape or k_cache.shape[1] != hk or \
            k_cache.shape[3] != hd:
        raise ValueError("store_kvcache_hnd: caches must be [num_blocks, Hk, page_size, D]")
    page = k_cache.shape[2] if page_size is None else int(page_size)
    if page != k_cache.shape[2]:
        raise ValueError(f"store_kvcache_hnd: page_size {page} != cache dim 2 "
                         f"({k_cache.shape[2]})")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("store_kvcache_hnd: caches must be contiguous")
    if not (key.dtype == value.dtype == k_cache.dtype == v_cache.dtype):
        raise TypeError("store_kvcache_hnd: key, value and both caches must share a dtype")
    if key.element_size() not in (1, 2, 4):
        raise TypeError(f"store_kvcache_hnd: element size {key.element_size()} unsupported")
    for t, nm in ((key, "key"), (value, "value")):
        if t.stride(2) != 1 or (hk > 1 and t.stride(1) != hd):
            raise ValueError(f"store_kvcache_hnd: {nm} rows must be [Hk, D] contiguous")
    if slot_mapping.dtype not in (torch.int32, torch.int64) or not slot_mapping.is_contiguous():
        raise TypeError("store_kvcache_hnd: slot_mapping must be contiguous int32 or int64")
    if slot_mapping.numel() < n:
        raise ValueError("store_kvcache_hnd: slot_mapping shorter than the token count")
    _same_device(key, value, k_cache, v_cache, slot_mapping)
    if n == 0:
        return
    _native.call("fk_store_kvcache_hnd", _ptr(key), key.stride(0), _ptr(value), value.stride(0),
                 _ptr(k_cache), _ptr(v_cache), _ptr(slot_mapping),
                 int(slot_mapping.dtype == torch.int64), n, hk, hd, page, key.element_size(),
                 k_cache.shape[0] * page, _stream(key))

# ---------------------------------------------------------------------------
# Fused per-head q/k RMSNorm + rotary + store_kvcache
# ---------------------------------------------------------------------------
def _token_rows(t: torch.Tensor, tokens: int, head_size: int, what: str) -> tuple[int, int]:
    """(row_stride, heads) of a [tokens, heads*head_size] (or [tokens, heads, head_size])
    view whose rows are contiguous."""
    w = t.numel() // tokens
    if w % head_size:
        raise ValueError(f"{what}: width {w} is not a multiple of head_size {head_size}")
    try:
        t2 = t.view(tokens, w)
    except RuntimeError as e:
        raise ValueError(f"{what}: rows must be [heads*head_size] ({e})") from None
    if t2.stride(1) != 1:
        raise ValueError(f"{what}: rows must be contiguous")
    return t2.stride(0), w // head_size


def qk_norm_rope_store(positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor,
                       value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                       slot_mapping: torch.Tensor, head_size: int, cos_sin_cache: torch.Tensor,
                       is_neox: bool, q_weight: torch.Tensor | None = None,
                       k_weight: torch.Tensor | None = None, eps: float = 1e-6) -> None:
    """One launch for: q = q_norm(q per head), k = k_norm(k per head) (when weights are
    given, Qwen3), rotary(positions, q, k), store_kvcache(k, v, caches, slot_mapping).

    query / key are rewritten in place (normed and rotated); the caches receive the
    rotated k rows and the v rows.  Bit-identical to rms_norm on each head row,
    rotary_embedding and store_kvcache run one after another."""
    if positions.dtype != torch.int64 or not positions.is_contiguous():
        raise TypeError("qk_norm_rope_store: positions must be contiguous int64")
    tokens = positions.numel()
    for t, nm in ((key, "key"), (value, "value"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        if t.dtype != query.dtype:
            raise TypeError(f"qk_norm_rope_store: {nm} dtype must equal the query dtype")
    if cos_sin_cache.dim() != 2 or not cos_sin_cache.is_contiguous() or \
            cos_sin_cache.dtype not in (torch.float32, query.dtype):
        raise ValueError("qk_norm_rope_store: cos_sin_cache must be contiguous float32 or "
                         "query-dtype [max_pos, rot_dim]")
    if (q_weight is None) != (k_weight is None):
        raise ValueError("qk_norm_rope_store: pass both q_weight and k_weight, or neither")
    for w, nm in ((q_weight, "q_weight"), (k_weight, "k_weight")):
        if w is not None and (w.dtype != query.dtype or w.numel() != head_size or
                              not w.is_contiguous()):
            raise ValueError(f"qk_norm_rope_store: {nm} must be contiguous [head_size] of the "
                             "query dtype")
    if slot_mapping.dtype not in (torch.int32, torch.int64) or not slot_mapping.is_contiguous() \
            or slot_mapping.numel() < tokens:
        raise TypeError("qk_norm_rope_store: slot_mapping must be contiguous int32/int64 [T]")
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape or k_cache.shape[3] != head_size \
            or not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("qk_norm_rope_store: caches must be contiguous [blocks, bs, Hk, D]")
    _same_device(positions, query, key, value, k_cache, v_cache, slot_mapping, cos_sin_cache)
    if tokens == 0:
        return
    qs, hq = _token_rows(query, tokens, head_size, "qk_norm_rope_store query")
    ks, hk = _token_rows(key, tokens, head_size, "qk_norm_rope_store key")
    vs, hv = _token_rows(value, tokens, head_size, "qk_norm_rope_store value")
    if hv != hk or k_cache.shape[2] != hk:
        raise ValueError("qk_norm_rope_store: key, value and caches must have the same kv heads")
    _native.call("fk_qk_norm_rope_store", _ptr(positions), _ptr(query), qs, _ptr(key), ks,
                 _ptr(value), vs, _ptr(q_weight), _ptr(k_weight), float(eps),
                 _ptr(cos_sin_cache), _tag(cos_sin_cache, "rotary cache"),
                 cos_sin_cache.shape[0], cos_sin_cache.shape[1], int(bool(is_neox)),
                 _ptr(k_cache), _ptr(v_cache), _ptr(slot_mapping),
                 int(slot_mapping.dtype == torch.int64), k_cache.shape[0] * k_cache.shape[1],
                 tokens, hq, hk, head_size, _tag(query, "qk_norm_rope_store"), _stream(query))


# ---------------------------------------------------------------------------
# Paged decode attention
# ---------------------------------------------------------------------------
class DecodePlan(NamedTuple):
    """Schedule of a paged-decode launch (fk_paged_decode_plan)."""
    part_tokens: int      # 0 = length-balanced schedule, else fixed partition size
    max_parts: int        # work-groups per kv-head group (balanced) / partitions per sequence
    workspace_bytes: int  # device workspace the launch needs


def paged_decode_plan(batch: int, num_heads: int, num_kv_heads: int, head_size: int,
                      max_seq_len: int, num_splits: int = 0) -> DecodePlan:
    """Plan a launch over contexts of at most max_seq_len.  num_splits = 0 picks the
    length-balanced schedule; num_splits > 0 asks for that many fixed partitions."""
    return DecodePlan(*_native.plan(batch, num_heads, num_kv_heads, head_size, max_seq_len,
                                    num_splits))


def _check_decode(out, q, k_cache, v_cache, block_table, cache_seqlens, k_scale, v_scale,
                  window_left=-1, sinks=None):
    if q.dim() != 3 or q.dtype != torch.bfloat16 or q.stride(2) != 1 or q.stride(1) != q.shape[2]:
        raise ValueError("paged_decode: q must be bf16 [B, Hq, D] with contiguous heads")
    b, hq, d = q.shape
    if out.shape != q.shape or out.dtype != q.dtype or out.stride(2) != 1 or out.stride(1) != d:
        raise ValueError("paged_decode: out must be bf16 [B, Hq, D] with contiguous heads")
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape or k_cache.shape[3] != d:
        raise ValueError("paged_decode: caches must be [num_blocks, block_size, Hk, D]")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("paged_decode: caches must be contiguous")
    if k_cache.dtype != v_cache.dtype or k_cache.dtype not in (torch.bfloat16, _FP8):
        raise TypeError("paged_decode: caches must both be bf16 or float8_e4m3fn")
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.stride(1) != 1:
        raise TypeError("paged_decode: block_table must be int32 [B, max_blocks], rows contiguous")
    if block_table.shape[0] < b:
        raise ValueError("paged_decode: block_table has fewer rows than the batch")
    if cache_seqlens.dtype != torch.int32 or not cache_seqlens.is_contiguous() or \
            cache_seqlens.numel() < b:
        raise TypeError("paged_decode: cache_seqlens must be contiguous int32 [B]")
    hk = k_cache.shape[2]
    for s, nm in ((k_scale, "k_scale"), (v_scale, "v_scale")):
        if s is not None and (s.dtype != torch.float32 or s.numel() != hk or
                              not s.is_contiguous()):
            raise ValueError(f"paged_decode: {nm} must be float32 [num_kv_heads]")
    if int(window_left) < -1:
        raise ValueError("paged_decode: window_left must be -1 (no window) or >= 0")
    if sinks is not None:
        if sinks.dtype != torch.float32 or sinks.numel() != hq or not sinks.is_contiguous():
            raise ValueError("paged_decode: sinks must be contiguous float32 [num_heads]")
        _same_device(q, sinks)
    _same_device(out, q, k_cache, v_cache, block_table, cache_seqlens)


def paged_decode(out: torch.Tensor, q: torch.Tensor, k_cache: torch.Tensor,
                 v_cache: torch.Tensor, block_table: torch.Tensor, cache_seqlens: torch.Tensor,
                 softmax_scale: float, part_tokens: int, max_parts: int,
                 workspace: torch.Tensor | None, k_scale: torch.Tensor | None = None,
                 v_scale: torch.Tensor | None = None, window_left: int = -1,
                 sinks: torch.Tensor | None = None) -> None:
    """Paged decode attention into ``out`` ([B, Hq, D] bf16).  window_left >= 0 limits
    each sequence to its last window_left + 1 keys (flash-attn window_size =
    (window_left, 0)); sinks (float32 [Hq], flash-attn s_aux) join each row's softmax
    denominator."""
    _check_decode(out, q, k_cache, v_cache, block_table, cache_seqlens, k_scale, v_scale,
                  window_left, sinks)
    b, hq, d = q.shape
    if b == 0:
        return
    nb, bs, hk, _ = k_cache.shape
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _native.call("fk_paged_decode", _ptr(out), out.stride(0), _ptr(q), q.stride(0),
                 _ptr(k_cache), _ptr(v_cache),
                 _native.FK_DTYPE_FP8_E4M3FN if k_cache.dtype == _FP8 else _native.FK_DTYPE_BF16,
                 _ptr(k_scale), _ptr(v_scale), _ptr(block_table), block_table.stride(0),
                 _ptr(cache_seqlens), b, hq, hk, d, bs, nb, float(softmax_scale),
                 int(window_left), _ptr(sinks), part_tokens, max_parts, _ptr(workspace),
                 ws_bytes, _stream(q))


def store_paged_decode(out: torch.Tensor, q: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                       k_cache: torch.Tensor, v_cache: torch.Tensor, slot_mapping: torch.Tensor,
                       block_table: torch.Tensor, cache_seqlens: torch.Tensor,
                       softmax_scale: float, part_tokens: int, max_parts: int,
                       workspace: torch.Tensor | None, k_scale: torch.Tensor | None = None,
                       v_scale: torch.Tensor | None = None, window_left: int = -1,
                       sinks: torch.Tensor | None = None) -> None:
    """store_kvcache(key, value, k_cache, v_cache, slot_mapping) followed by
    paged_decode(...) in one launch (plus the merge launch).

    Decode step layout: token b is sequence b's new token, so key/value/slot_mapping
    have B rows and slot_mapping[b] is -1 or the slot of position cache_seqlens[b] - 1
    in block_table[b] (fastkernels/infra/engine.py:5020-5024).  The result then equals
    the two separate calls bit for bit.  Other slots are still written, but the
    attention output of a sequence that reads another token's slot is unspecified."""
    _check_decode(out, q, k_cache, v_cache, block_table, cache_seqlens, k_scale, v_scale,
                  window_left, sinks)
    b, hq, d = q.shape
    nb, bs, hk, _ = k_cache.shape
    if key.shape != (b, hk, d) or value.shape != key.shape:
        raise ValueError("store_paged_decode: key/value must be [B, num_kv_heads, head_dim]")
    if key.dtype != k_cache.dtype or value.dtype != v_cache.dtype:
        raise TypeError("store_paged_decode: key/value dtype must equal the cache dtype")
    for t, nm in ((key, "key"), (value, "value")):
        if t.stride(2) != 1 or (hk > 1 and t.stride(1) != d):
            raise ValueError(f"store_paged_decode: {nm} rows must be [Hk, D] contiguous")
    if slot_mapping.dtype not in (torch.int32, torch.int64) or not slot_mapping.is_contiguous() \
            or slot_mapping.numel() < b:
        raise TypeError("store_paged_decode: slot_mapping must be contiguous int32/int64 [B]")
    _same_device(q, key, value, slot_mapping)
    if b == 0:
        return
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _native.call("fk_store_paged_decode", _ptr(out), out.stride(0), _ptr(q), q.stride(0),
                 _ptr(key), key.stride(0), _ptr(value), value.stride(0), _ptr(slot_mapping),
                 int(slot_mapping.dtype == torch.int64), _ptr(k_cache), _ptr(v_cache),
                 _native.FK_DTYPE_FP8_E4M3FN if k_cache.dtype == _FP8 else _native.FK_DTYPE_BF16,
                 _ptr(k_scale), _ptr(v_scale), _ptr(block_table), block_table.stride(0),
                 _ptr(cache_seqlens), b, hq, hk, d, bs, nb, float(softmax_scale),
                 int(window_left), _ptr(sinks), part_tokens, max_parts, _ptr(workspace),
                 ws_bytes, _stream(q))


def _check_prefill_extras(q, causal, window_left, sinks):
    if int(window_left) < -1:
        raise ValueError("prefill: window_left must be -1 (no window) or >= 0")
    if int(window_left) >= 0 and not causal:
        raise ValueError("prefill: a sliding window needs causal attention")
    if sinks is not None:
        if sinks.dtype != torch.float32 or sinks.numel() != q.shape[1] or \
                not sinks.is_contiguous():
            raise ValueError("prefill: sinks must be contiguous float32 [num_heads]")
        _same_device(q, sinks)


# (query / key, value) head sizes the prefill kernel is built for (fp8 pages: the
# equal sizes 64, 128 and 256).
PREFILL_HEADS = {(32, 32), (64, 64), (72, 72), (80, 80), (96, 96), (128, 128), (256, 256),
                 (192, 128)}
PREFILL_FP8_HEADS = {(64, 64), (128, 128), (256, 256)}


def prefill_heads_supported(head_size: int, head_size_v: int | None = None,
                            fp8: bool = False) -> bool:
    """Whether the prefill kernel runs at these query / key and value head sizes."""
    pair = (int(head_size), int(head_size if head_size_v is None else head_size_v))
    return pair in (PREFILL_FP8_HEADS if fp8 else PREFILL_HEADS)


def _check_prefill(out, q, cu_seqlens_q, cu_seqlens_k, dv=None):
    dv = q.shape[2] if dv is None else dv
    if q.dim() != 3 or q.dtype != torch.bfloat16 or q.stride(2) != 1 or q.stride(1) != q.shape[2]:
        raise ValueError("prefill: q must be bf16 [tokens, Hq, D] with contiguous heads")
    if tuple(out.shape) != (q.shape[0], q.shape[1], dv) or out.dtype != q.dtype or \
            out.stride(2) != 1 or out.stride(1) != dv:
        raise ValueError("prefill: out must be bf16 [tokens, Hq, Dv] with contiguous heads")
    for t, nm in ((cu_seqlens_q, "cu_seqlens_q"), (cu_seqlens_k, "cu_seqlens_k")):
        if t.dtype != torch.int32 or t.dim() != 1 or not t.is_contiguous():
            raise TypeError(f"prefill: {nm} must be contiguous int32 [batch + 1]")
    if cu_seqlens_k.numel() < cu_seqlens_q.numel():
        raise ValueError("prefill: cu_seqlens_k shorter than cu_seqlens_q")


def _check_lse(lse, q, what):
    if lse is None:
        return
    if lse.dtype != torch.float32 or lse.dim() != 2 or lse.shape[0] != q.shape[1] or \
            lse.shape[1] < q.shape[0] or lse.stride(1) != 1:
        raise ValueError(f"{what}: lse must be float32 [num_heads, >= total_q] with "
                         "contiguous rows")
    _same_device(q, lse)


# Work-group key split of the prefill: False launches without it (the library's
# plain launch, for A/B timing and the tests that compare the two).
PREFILL_SPLIT = True


def _split_workspace(q, paged, kv_dtype, batch, max_seqlen_q, max_seqlen_k, hk, dv, causal):
    """The workspace of the prefill's work-group key split (fk_prefill_split_plan), from
    torch's allocator on q's stream, or None when the launch does not split."""
    if not PREFILL_SPLIT:
        return None
    nbytes = _native.prefill_split_bytes(paged, kv_dtype, batch, q.shape[0], int(max_seqlen_q),
                                         int(max_seqlen_k), q.shape[1], hk, q.shape[2], dv,
                                         causal)
    return torch.empty(nbytes, dtype=torch.uint8, device=q.device) if nbytes > 0 else None


def paged_prefill(out: torch.Tensor, q: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, block_table: torch.Tensor, cu_seqlens_q: torch.Tensor,
                  cu_seqlens_k: torch.Tensor, max_seqlen_q: int, softmax_scale: float,
                  k_scale: torch.Tensor | None = None, v_scale: torch.Tensor | None = None,
                  causal: bool = True, window_left: int = -1,
                  sinks: torch.Tensor | None = None, max_seqlen_k: int = 0) -> None:
    """Causal prefill over paged K/V into ``out`` ([tokens, Hq, Dv] bf16): sequence b's
    queries q[cu_q[b]:cu_q[b+1]] attend to its first cu_k[b+1]-cu_k[b] cached tokens,
    aligned to their end (flash_attn_varlen_func with block_table, seqused_k).
    window_left >= 0: each query sees its last window_left + 1 positions; sinks
    (float32 [Hq]) join each row's softmax denominator.  max_seqlen_k bounds every
    sequence's key count (0: unknown); it only chooses the launch shape.  The value
    cache may have its own head size Dv (``PREFILL_HEADS``)."""
    dv = v_cache.shape[3] if v_cache.dim() == 4 else q.shape[2]
    _check_prefill(out, q, cu_seqlens_q, cu_seqlens_k, dv)
    _check_prefill_extras(q, causal, window_left, sinks)
    if k_cache.dim() != 4 or v_cache.dim() != 4 or v_cache.shape[:3] != k_cache.shape[:3] or \
            k_cache.shape[3] != q.shape[2]:
        raise ValueError("paged_prefill: caches must be [num_blocks, block_size, Hk, D] "
                         "(the value cache's head size may differ)")
    if not prefill_heads_supported(q.shape[2], dv, k_cache.dtype == _FP8):
        raise NotImplementedError(f"paged_prefill: head sizes {q.shape[2]} / {dv} are not "
                                  "built (see ops.PREFILL_HEADS)")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("paged_prefill: caches must be contiguous")
    if k_cache.dtype != v_cache.dtype or k_cache.dtype not in (torch.bfloat16, _FP8):
        raise TypeError("paged_prefill: caches must both be bf16 or float8_e4m3fn")
    batch = cu_seqlens_q.numel() - 1
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.stride(1) != 1 \
            or block_table.shape[0] < batch:
        raise TypeError("paged_prefill: block_table must be int32 [batch, max_blocks], rows "
                        "contiguous")
    hk = k_cache.shape[2]
    for sc, nm in ((k_scale, "k_scale"), (v_scale, "v_scale")):
        if sc is not None and (sc.dtype != torch.float32 or sc.numel() != hk or
                               not sc.is_contiguous()):
            raise ValueError(f"paged_prefill: {nm} must be float32 [num_kv_heads]")
    _same_device(out, q, k_cache, v_cache, block_table, cu_seqlens_q, cu_seqlens_k)
    if batch <= 0 or q.shape[0] == 0:
        return
    nb, bs = k_cache.shape[:2]
    kv_dtype = _native.FK_DTYPE_FP8_E4M3FN if k_cache.dtype == _FP8 else _native.FK_DTYPE_BF16
    ws = _split_workspace(q, True, kv_dtype, batch, max_seqlen_q, max_seqlen_k, hk, dv, causal)
    _native.call("fk_paged_prefill_ws", _ptr(out), out.stride(0), _ptr(q), q.stride(0),
                 _ptr(k_cache), _ptr(v_cache), kv_dtype,
                 _ptr(k_scale), _ptr(v_scale), _ptr(block_table), block_table.stride(0),
                 _ptr(cu_seqlens_q), _ptr(cu_seqlens_k), batch, int(max_seqlen_q),
                 int(max_seqlen_k), q.shape[1], hk, q.shape[2], dv, bs, nb,
                 float(softmax_scale), int(bool(causal)), int(window_left), _ptr(sinks),
                 q.shape[0], _ptr(ws), 0 if ws is None else ws.numel(), _stream(q))


def varlen_prefill(out: torch.Tensor, q: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                   cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor, max_seqlen_q: int,
                   softmax_scale: float, causal: bool = True, window_left: int = -1,
                   sinks: torch.Tensor | None = None, max_seqlen_k: int = 0,
                   lse: torch.Tensor | None = None) -> None:
    """Causal prefill over dense keys: key [total_k, Hk, D] / value [total_k, Hk, Dv] bf16
    (rows may be strided views), sequence b's keys being rows cu_k[b]..cu_k[b+1].
    window_left, sinks, max_seqlen_k and head sizes as in :func:`paged_prefill`.  lse
    (float32 [Hq, >= total_q], rows contiguous) receives each row's softmax log-sum-exp,
    -inf without visible keys (FlashAttnVarlen's return_softmax_lse,
    flash_attn_varlen.py:21-47)."""
    dv = value.shape[2] if value.dim() == 3 else q.shape[2]
    _check_prefill(out, q, cu_seqlens_q, cu_seqlens_k, dv)
    _check_prefill_extras(q, causal, window_left, sinks)
    _check_lse(lse, q, "varlen_prefill")
    if key.dim() != 3 or value.dim() != 3 or value.shape[:2] != key.shape[:2] or \
            key.shape[2] != q.shape[2]:
        raise ValueError("varlen_prefill: key must be [total_k, Hk, D] and value "
                         "[total_k, Hk, Dv]")
    if not prefill_heads_supported(q.shape[2], dv):
        raise NotImplementedError(f"varlen_prefill: head sizes {q.shape[2]} / {dv} are not "
                                  "built (see ops.PREFILL_HEADS)")
    for t, nm in ((key, "key"), (value, "value")):
        if t.dtype != torch.bfloat16 or t.stride(2) != 1 or (t.shape[1] > 1 and
                                                             t.stride(1) != t.shape[2]):
            raise ValueError(f"varlen_prefill: {nm} must be bf16 with [Hk, D] contiguous rows")
    _same_device(out, q, key, value, cu_seqlens_q, cu_seqlens_k)
    batch = cu_seqlens_q.numel() - 1
    if batch <= 0 or q.shape[0] == 0:
        return
    ws = _split_workspace(q, False, _native.FK_DTYPE_BF16, batch, max_seqlen_q, max_seqlen_k,
                          key.shape[1], dv, causal)
    _native.call("fk_varlen_prefill_ws", _ptr(out), out.stride(0), _ptr(q), q.stride(0),
                 _ptr(key), key.stride(0), _ptr(value), value.stride(0), _ptr(cu_seqlens_q),
                 _ptr(cu_seqlens_k), batch, int(max_seqlen_q), int(max_seqlen_k), q.shape[1],
                 key.shape[1], q.shape[2], dv, float(softmax_scale), int(bool(causal)),
                 int(window_left), _ptr(sinks), _ptr(lse), 0 if lse is None else lse.stride(0),
                 q.shape[0], _ptr(ws), 0 if ws is None else ws.numel(), _stream(q))


def paged_decode_phases(out, q, k_cache, v_cache, block_table, cache_seqlens, softmax_scale,
                        part_tokens, max_parts, workspace, k_scale=None, v_scale=None,
                        window_left=-1, sinks=None):
    """The two launches of :func:`paged_decode` as separate callables (for timing)."""
    _check_decode(out, q, k_cache, v_cache, block_table, cache_seqlens, k_scale, v_scale,
                  window_left, sinks)
    b, hq, d = q.shape
    nb, bs, hk, _ = k_cache.shape
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    kvd = _native.FK_DTYPE_FP8_E4M3FN if k_cache.dtype == _FP8 else _native.FK_DTYPE_BF16
    stream = _stream(q)
    lib = _native.lib()
    part_args = (_ptr(out), out.stride(0), _ptr(q), q.stride(0), _ptr(k_cache), _ptr(v_cache),
                 kvd, _ptr(k_scale), _ptr(v_scale), _ptr(block_table), block_table.stride(0),
                 _ptr(cache_seqlens), b, hq, hk, d, bs, nb, float(softmax_scale),
                 int(window_left), _ptr(sinks), part_tokens, max_parts, _ptr(workspace), ws_bytes,
                 stream)
    fp, fr = lib.fk_paged_decode_partials, lib.fk_paged_decode_reduce

    def partials():
        _native.check("fk_paged_decode_partials", fp(*part_args))

    def reduce():
        _native.check("fk_paged_decode_reduce", fr(*part_args))

    return partials, reduce


# ---------------------------------------------------------------------------
# SiLU-and-mul
# ---------------------------------------------------------------------------
def silu_and_mul(out: torch.Tensor, x: torch.Tensor) -> None:
    """out = silu(x[..., :d]) * x[..., d:] (``_C.silu_and_mul(out, x)`` contract)."""
    d = x.shape[-1] // 2
    if x.shape[-1] != 2 * d or out.shape != x.shape[:-1] + (d,) or out.dtype != x.dtype:
        raise ValueError("silu_and_mul: out must be x.shape[:-1] + (d,) with x's dtype")
    _same_device(out, x)
    rows, xs = _rows(x, 2 * d, "silu_and_mul x")
    _, os_ = _rows(out, d, "silu_and_mul out")
    if rows == 0 or d == 0:
        return
    _native.call("fk_silu_and_mul", _ptr(out), os_, _ptr(x), xs, rows, d, _tag(x, "silu_and_mul"),
                 _stream(x))


# ---------------------------------------------------------------------------
# merge_attn_states
# ---------------------------------------------------------------------------
def merge_attn_states(output: torch.Tensor, prefix_output: torch.Tensor, prefix_lse: torch.Tensor,
                      suffix_output: torch.Tensor, suffix_lse: torch.Tensor,
                      output_lse: torch.Tensor | None = None,
                      prefill_tokens_with_context: int | None = None,
                      output_scale: torch.Tensor | None = None) -> None:
    """LSE merge of two partial attention results into ``output`` (and ``output_lse``).

    output / prefix_output / suffix_output: [T, H, D] (D contiguous; prefix and suffix
    share strides); *_lse: float32 [H, T], natural log.  An ``output`` of
    float8_e4m3fn takes ``output_scale`` (float32, one element): every output value
    becomes e4m3fn(clamp(v / output_scale, -448, 448)) (merge_attn_states.cu's
    USE_FP8_OUTPUT form)."""
    if prefix_output.stride(1) != suffix_output.stride(1) or \
            prefix_output.stride(0) != suffix_output.stride(0):
        raise ValueError("merge_attn_states: prefix_output and suffix_output must share strides")
    if output.dim() != 3 or prefix_output.shape != output.shape or suffix_output.shape != output.shape:
        raise ValueError("merge_attn_states: outputs must be [tokens, heads, head_size]")
    if suffix_output.dtype != prefix_output.dtype:
        raise TypeError("merge_attn_states: prefix and suffix must share a dtype")
    fp8_out = output.dtype == _FP8
    if fp8_out:
        if output_scale is None:
            raise ValueError(f"merge_attn_states: output_scale is required when output is "
                             f"{output.dtype}")
        if output_scale.dtype != torch.float32 or output_scale.numel() != 1:
            raise ValueError("merge_attn_states: output_scale must be one float32 value")
        _same_device(output, output_scale)
    elif output.dtype != prefix_output.dtype:
        raise TypeError("merge_attn_states: output must be the inputs' dtype or float8_e4m3fn")
    t, h, d = output.shape
    for x in (output, prefix_output, suffix_output):
        if x.stride(2) != 1:
            raise ValueError("merge_attn_states: head_size must be contiguous")
    for x, nm in ((prefix_lse, "prefix_lse"), (suffix_lse, "suffix_lse"), (output_lse, "output_lse")):
        if x is not None and (x.dtype != torch.float32 or tuple(x.shape) != (h, t) or
                              not x.is_contiguous()):
            raise ValueError(f"merge_attn_states: {nm} must be contiguous float32 [heads, tokens]")
    _same_device(output, prefix_output, suffix_output, prefix_lse, suffix_lse)
    if t == 0 or h == 0:
        return
    in_tag = _tag(prefix_output, "merge_attn_states")
    _native.call("fk_merge_attn_states", _ptr(output), output.stride(0), output.stride(1),
                 _ptr(output_lse), _ptr(prefix_output), _ptr(prefix_lse), _ptr(suffix_output),
                 _ptr(suffix_lse), prefix_output.stride(0), prefix_output.stride(1), t, h, d,
                 -1 if prefill_tokens_with_context is None else int(prefill_tokens_with_context),
                 in_tag, _native.FK_DTYPE_FP8_E4M3FN if fp8_out else in_tag,
                 _ptr(output_scale if fp8_out else None), _stream(output))


# ---------------------------------------------------------------------------
# torch.library registration (opaque custom ops with mutation annotations).
# ---------------------------------------------------------------------------
_LIB = torch.library.Library("fastkernels_amd", "DEF")
_LIB.define("rmsnorm(Tensor! result, Tensor input, Tensor weight, float eps) -> ()")
_LIB.define("fused_add_rmsnorm(Tensor(a!) input, Tensor(b!) residual, Tensor weight, "
            "float eps) -> ()")
_LIB.define("rotary_embedding(Tensor positions, Tensor(a!) query, Tensor(b!)? key, "
            "int head_size, Tensor cos_sin_cache, bool is_neox) -> ()")
_LIB.define("store_kvcache(Tensor key, Tensor value, Tensor(a!) k_cache, Tensor(b!) v_cache, "
            "Tensor slot_mapping) -> ()")
_LIB.define("store_kvcache_hnd(Tensor key, Tensor value, Tensor(a!) k_cache, Tensor(b!) v_cache, "
            "Tensor slot_mapping, int? page_size=None) -> ()")
_LIB.define("paged_decode(Tensor(a!) out, Tensor q, Tensor k_cache, Tensor v_cache, "
            "Tensor block_table, Tensor cache_seqlens, float softmax_scale, int part_tokens, "
            "int max_parts, Tensor(b!)? workspace, Tensor? k_scale, Tensor? v_scale, "
            "int window_left=-1, Tensor? sinks=None) -> ()")
_LIB.define("store_paged_decode(Tensor(a!) out, Tensor q, Tensor key, Tensor value, "
            "Tensor(b!) k_cache, Tensor(c!) v_cache, Tensor slot_mapping, Tensor block_table, "
            "Tensor cache_seqlens, float softmax_scale, int part_tokens, int max_parts, "
            "Tensor(d!)? workspace, Tensor? k_scale=None, Tensor? v_scale=None, "
            "int window_left=-1, Tensor? sinks=None) -> ()")
_LIB.define("qk_norm_rope_store(Tensor positions, Tensor(a!) query, Tensor(b!) key, "
            "Tensor value, Tensor(c!) k_cache, Tensor(d!) v_cache, Tensor slot_mapping, "
            "int head_size, Tensor cos_sin_cache, bool is_neox, Tensor? q_weight=None, "
            "Tensor? k_weight=None, float eps=1e-6) -> ()")
_LIB.define("paged_prefill(Tensor(a!) out, Tensor q, Tensor k_cache, Tensor v_cache, "
            "Tensor block_table, Tensor cu_seqlens_q, Tensor cu_seqlens_k, int max_seqlen_q, "
            "float softmax_scale, Tensor? k_scale=None, Tensor? v_scale=None, bool causal=True, "
            "int window_left=-1, Tensor? sinks=None, int max_seqlen_k=0) -> ()")
_LIB.define("varlen_prefill(Tensor(a!) out, Tensor q, Tensor key, Tensor value, "
            "Tensor cu_seqlens_q, Tensor cu_seqlens_k, int max_seqlen_q, float softmax_scale, "
            "bool causal=True, int window_left=-1, Tensor? sinks=None, "
            "int max_seqlen_k=0, Tensor(b!)? lse=None) -> ()")
_LIB.define("silu_and_mul(Tensor! result, Tensor input) -> ()")
_LIB.define("merge_attn_states(Tensor(a!) output, Tensor prefix_output, Tensor prefix_lse, "
            "Tensor suffix_output, Tensor suffix_lse, Tensor(b!)? output_lse, "
            "int? prefill_tokens_with_context=None, Tensor? output_scale=None) -> ()")

_IMPLS = {
    "rmsnorm": lambda result, input, weight, eps: rms_norm(result, input, weight, eps),
    "fused_add_rmsnorm": fused_add_rms_norm,
    "rotary_embedding": rotary_embedding,
    "store_kvcache": store_kvcache,
    "store_kvcache_hnd": store_kvcache_hnd,
    "paged_decode": paged_decode,
    "silu_and_mul": lambda result, input: silu_and_mul(result, input),
    "merge_attn_states": merge_attn_states,
    "store_paged_decode": store_paged_decode,
    "qk_norm_rope_store": qk_norm_rope_store,
    "paged_prefill": paged_prefill,
    "varlen_prefill": varlen_prefill,
}
for _name, _fn in _IMPLS.items():
    _LIB.impl(_name, _fn, "CUDA")
    _LIB.impl(_name, lambda *a, **k: None, "Meta")


def default_softmax_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)
