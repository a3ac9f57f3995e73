"""CPU oracle for the decode-step operator path (numpy restatement of the reference).

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``fastkernels_amd``) imports,
links or calls this package.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg use it, and only as the checker (or as the
CPU baseline being timed), never as an implementation of an op.

Conventions: tensors are numpy arrays holding the *values* of the reference's
tensors as float32 (every bf16 / fp16 value is exactly a float32), plus a dtype
tag ("bf16", "f16", "f32") saying where the reference rounds.  ``round_to``
performs that rounding (round-to-nearest-even, as torch does).  fp8 KV caches
are uint8 arrays of OCP e4m3fn codes.

Each function names the reference code it restates (paths relative to the
Snowflake-AI-Research/fastkernels checkout).  How each is pinned (golden
vectors, library routines, closed forms, invariants, brute force) is listed in
tests/test_oracle.py; a function none of those pin would be marked
"parity unpinned" here — none is.
"""
from __future__ import annotations

import numpy as np

# ---------------------------------------------------------------------------
# Number formats
# ---------------------------------------------------------------------------


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float32 values (exact)."""
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round-to-nearest-even; NaN -> 0x7fc0."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16
    r = np.where(nan, np.uint32(0x7FC0), r)
    return r.astype(np.uint16)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float values to ``dtype`` and return them as float32."""
    x = np.asarray(x, np.float32)
    if dtype == "bf16":
        return bf16_bits_to_f32(f32_to_bf16_bits(x))
    if dtype == "f16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "f32":
        return x
    raise ValueError(f"unknown dtype {dtype}")


def _e4m3fn_table() -> np.ndarray:
    """Value of every OCP float8 e4m3fn code: 1 sign, 4 exponent (bias 7), 3 mantissa
    bits; exponent 0 is subnormal (m/8 * 2^-6); code S.1111.111 is NaN; no infinities."""
    t = np.empty(256, np.float32)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xF
        m = c & 0x7
        if e == 0xF and m == 0x7:
            t[c] = np.nan
        elif e == 0:
            t[c] = s * (m / 8.0) * 2.0 ** -6
        else:
            t[c] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return t


E4M3FN_TABLE = _e4m3fn_table()
E4M3FN_MAX = 448.0


def fp8_e4m3fn_decode(codes: np.ndarray) -> np.ndarray:
    return E4M3FN_TABLE[np.asarray(codes, np.uint8)]


def fp8_e4m3fn_encode(x: np.ndarray) -> np.ndarray:
    """Saturating round-to-nearest-even float -> e4m3fn code (|x| clamped to 448; NaN
    gives the NaN code with the input's sign), the conversion of a Triton tl.store into a
    float8e4nv pointer (round to nearest even, saturate to finite)."""
    x = np.asarray(x, np.float64)
    nan = np.isnan(x)
    sign = np.signbit(x).ravel()  # negative values that round to 0 give -0 (0x80)
    x = np.clip(np.where(nan, 0.0, x), -E4M3FN_MAX, E4M3FN_MAX)
    finite = E4M3FN_TABLE.astype(np.float64)
    pos_codes = np.arange(0, 0x7F, dtype=np.int64)  # 0 .. 0x7E are the finite non-negatives
    pos_vals = finite[pos_codes]
    a = np.abs(x).ravel()
    idx = np.searchsorted(pos_vals, a)  # pos_vals is increasing
    idx = np.clip(idx, 1, len(pos_vals) - 1)
    lo, hi = pos_vals[idx - 1], pos_vals[idx]
    pick_hi = (a - lo > hi - a) | ((a - lo == hi - a) & ((pos_codes[idx] & 1) == 0))
    code = np.where(pick_hi, pos_codes[idx], pos_codes[idx - 1])
    code = np.where(a == 0, 0, code)
    code = np.where(nan.ravel(), 0x7F, code)
    return (code | (sign.astype(np.int64) << 7)).astype(np.uint8).reshape(np.shape(x))


# ---------------------------------------------------------------------------
# RMSNorm — RMSNorm.forward_native, fastkernels/tasks/baseline/L1/rms_norm.py:97-118
# ---------------------------------------------------------------------------


def rms_norm(x: np.ndarray, weight: np.ndarray, eps: float, dtype: str,
             residual: np.ndarray | None = None):
    """Returns ``out`` (no residual) or ``(out, new_residual)``.

    xf = float(x) [+ float(residual)]; new_residual = cast(xf);
    var = mean(xf^2); out = cast(cast(xf * rsqrt(var + eps)) * weight)."""
    xf = np.asarray(x, np.float32)
    if residual is not None:
        xf = xf + np.asarray(residual, np.float32)
        new_res = round_to(xf, dtype)
    var = np.mean(xf.astype(np.float64) ** 2, axis=-1, keepdims=True)
    inv = (1.0 / np.sqrt(var + eps)).astype(np.float32)
    xh = round_to(xf * inv, dtype)
    out = round_to(xh * np.asarray(weight, np.float32), dtype)
    return out if residual is None else (out, new_res)


# ---------------------------------------------------------------------------
# Rotary — RotaryEmbedding, fastkernels/tasks/baseline/L1/rotary_emb.py:79-191
# ---------------------------------------------------------------------------


def rope_inv_freq(head_dim: int, theta: float) -> np.ndarray:
    """inv_freq_i = 1 / theta^(2i/D) (rotary_emb.py:93), in float32 as torch forms it."""
    exps = (np.arange(0, head_dim, 2, dtype=np.float32) / np.float32(head_dim)).astype(np.float32)
    return (np.float32(1.0) / np.power(np.float32(theta), exps, dtype=np.float32)).astype(np.float32)


def rope_cos_sin_cache(head_dim: int, max_pos: int, theta: float) -> np.ndarray:
    """[max_pos, head_dim] float32: cos(t * inv_freq) then sin(t * inv_freq) (:104-107)."""
    inv = rope_inv_freq(head_dim, theta)
    ang = np.outer(np.arange(max_pos, dtype=np.float32), inv).astype(np.float32)
    return np.concatenate([np.cos(ang), np.sin(ang)], axis=-1).astype(np.float32)


def rotary(positions: np.ndarray, query: np.ndarray, key: np.ndarray | None, head_size: int,
           cos_sin: np.ndarray, is_neox: bool, dtype: str):
    """Rotated copies of query/key ([T, H*D] values).  cos/sin are cast to the query
    dtype (rotary_emb.py:171-173); products and sums in fp32, one rounding."""
    pos = np.asarray(positions, np.int64)
    cs = round_to(np.asarray(cos_sin, np.float32)[pos], dtype)  # [T, rot]
    rot = cs.shape[-1]
    half = rot // 2
    cos, sin = cs[:, None, :half], cs[:, None, half:]

    def apply(x):
        t = x.shape[0]
        xh = np.asarray(x, np.float32).reshape(t, -1, head_size).copy()
        if is_neox:
            a, b = xh[..., :half].copy(), xh[..., half:rot].copy()
            xh[..., :half] = a * cos - b * sin
            xh[..., half:rot] = b * cos + a * sin
        else:
            a, b = xh[..., 0:rot:2].copy(), xh[..., 1:rot:2].copy()
            xh[..., 0:rot:2] = a * cos - b * sin
            xh[..., 1:rot:2] = b * cos + a * sin
        return round_to(xh, dtype).reshape(x.shape)

    return apply(query), (apply(key) if key is not None else None)


# ---------------------------------------------------------------------------
# store_kvcache — _store_kvcache_kernel, fastkernels/tasks/baseline/L1/store_kvcache.py:16-35
# ---------------------------------------------------------------------------


def store_kvcache_(key: np.ndarray, value: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                   slot_mapping: np.ndarray) -> None:
    """In-place scatter: for token i with s = slot_mapping[i] >= 0, cache row s = key[i]
    (the row is Hk*D elements; the cache viewed as [num_blocks * block_size, Hk*D])."""
    nb, bs = k_cache.shape[:2]
    kflat = k_cache.reshape(nb * bs, -1)
    vflat = v_cache.reshape(nb * bs, -1)
    slots = np.asarray(slot_mapping, np.int64)
    n = key.shape[0]
    keep = slots[:n] >= 0
    idx = slots[:n][keep]
    kflat[idx] = key.reshape(n, -1)[keep]
    vflat[idx] = value.reshape(n, -1)[keep]


def store_kvcache(key: np.ndarray, value: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                  slot_mapping: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Copies of the caches after the scatter.  Arrays may be any dtype (bit copy):
    key/value [N, Hk, D]; caches [num_blocks, block_size, Hk, D]; slot < 0 skips."""
    kc, vc = k_cache.copy(), v_cache.copy()
    store_kvcache_(key, value, kc, vc, slot_mapping)
    return kc, vc


# ---------------------------------------------------------------------------
# Paged decode attention — Attention._decode_torch / _cache_seq / _sdpa_one /
# _repeat_kv_for_heads, fastkernels/tasks/baseline/L2/attention_impl.py:592-664
# ---------------------------------------------------------------------------


def store_kvcache_hnd(key: np.ndarray, value: np.ndarray, k_cache: np.ndarray,
                      v_cache: np.ndarray, slot_mapping: np.ndarray, page_size: int):
    """StoreKVCacheHND (store_kvcache.py:36-68, 85-99) on copies of the caches:
    caches [num_blocks, Hk, page_size, D]; token i's head h row goes to
    cache[s // page_size, h, s % page_size] for s = slot_mapping[i] >= 0 (and, as the
    kernel does, slots past the cache are skipped)."""
    kc, vc = k_cache.copy(), v_cache.copy()
    nslots = kc.shape[0] * page_size
    for i, s in enumerate(np.asarray(slot_mapping, np.int64)[:key.shape[0]]):
        if s < 0 or s >= nslots:
            continue
        kc[s // page_size, :, s % page_size] = key[i]
        vc[s // page_size, :, s % page_size] = value[i]
    return kc, vc


def gather_seq(cache: np.ndarray, block_row: np.ndarray, length: int) -> np.ndarray:
    """_cache_seq (attention_impl.py:598-604): the first `length` token rows of a sequence."""
    bs = cache.shape[1]
    pages = (length + bs - 1) // bs
    ids = np.asarray(block_row[:pages], np.int64)
    return cache[ids].reshape(-1, cache.shape[2], cache.shape[3])[:length]


def dequant_kv(cache: np.ndarray, scale: np.ndarray | None, q_dtype: str) -> np.ndarray:
    """fp8 per-(kv head) dequant: cast(float(x) * scale) to the query dtype
    (_cast_kv_tile, triton_unified_attention.py:64-67).  Non-fp8 caches pass through.
    `scale` is one value per kv head, or a single per-tensor value (the reference's
    FP8_PER_TENSOR mode, kv_quant_mode.py:20) broadcast to every head."""
    if cache.dtype != np.uint8:
        return np.asarray(cache, np.float32)
    hk = cache.shape[2]
    if scale is None:
        sc = np.ones(hk, np.float32)
    else:
        sc = np.asarray(scale, np.float32).reshape(-1)
        if sc.size == 1:
            sc = np.full(hk, sc[0], np.float32)
        elif sc.size != hk:
            raise ValueError(f"dequant_kv: {sc.size} scales for {hk} kv heads")
    # The value is a function of (code, kv head) only: tabulate round(decode(c) * s_h)
    # for the 256 codes of each head, then gather (the same values, one pass).
    tables = round_to(E4M3FN_TABLE[None, :] * sc[:, None], q_dtype)  # [Hk, 256]
    out = np.empty(cache.shape, np.float32)
    for h in range(hk):
        out[:, :, h, :] = tables[h][cache[:, :, h, :]]
    return out


def attend_one(q: np.ndarray, k_seq: np.ndarray, v_seq: np.ndarray, scale: float,
               sinks: np.ndarray | None = None) -> np.ndarray:
    """softmax(scale * q k^T) v for one query token; GQA by head // (Hq/Hk)
    (repeat_interleave, attention_impl.py:592-596).  float64; 0 rows when empty.

    sinks ([Hq], the flash-attn ``s_aux`` logits, in the units of scale * q.k) join
    the denominator only: the online softmax starts from M = sink, L = 1
    (init_softmax_M, fastkernels/infra/triton_attention_helpers.py) and the
    split-K reduce adds the sink once (reduce_segments,
    triton_unified_attention.py:741-776), so a row is
    sum_t e^(s_t - m) v_t / (sum_t e^(s_t - m) + e^(sink - m))."""
    hq, d = q.shape
    n, hk, _ = k_seq.shape
    if n == 0:
        return np.zeros((hq, d), np.float64)
    grp = hq // hk
    qh = q.astype(np.float64).reshape(hk, grp, d)
    sk = None if sinks is None else np.asarray(sinks, np.float64).reshape(hk, grp, 1)
    out = np.empty((hk, grp, d), np.float64)
    for h in range(hk):  # one kv head at a time: contiguous [n, D] operands, 2-D products
        k = np.ascontiguousarray(k_seq[:, h, :], np.float64)
        v = np.ascontiguousarray(v_seq[:, h, :], np.float64)
        s = (qh[h] @ k.T) * scale  # [grp, n]
        m = s.max(axis=-1, keepdims=True)
        if sk is not None:
            m = np.maximum(m, sk[h])
        p = np.exp(s - m)
        den = p.sum(axis=-1, keepdims=True)
        if sk is not None:
            den = den + np.exp(sk[h] - m)
        out[h] = (p / den) @ v
    return out.reshape(hq, d)


def paged_decode(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                 block_tables: np.ndarray, ctx_lens: np.ndarray, scale: float,
                 k_scale: np.ndarray | None = None, v_scale: np.ndarray | None = None,
                 q_dtype: str = "bf16", seqs=None, window_left: int = -1,
                 sinks: np.ndarray | None = None) -> np.ndarray:
    """Decode attention output [B, Hq, D] (float64, unrounded) — `_decode_torch`.

    q: [B, Hq, D] values; caches [num_blocks, block_size, Hk, D] values, or uint8
    e4m3fn codes with per-kv-head scales.  ``seqs`` restricts the sequences
    computed (others stay 0), for bounded CPU-baseline samples.

    window_left >= 0 is a sliding window, flash-attn window_size = (window_left, 0):
    the query at position n - 1 sees keys [n - 1 - window_left, n - 1] (the
    SLIDING_WINDOW = 1 + window_size[0] mask of triton_unified_attention.py:577-590
    and :953).  sinks: see attend_one."""
    b, hq, d = q.shape
    out = np.zeros((b, hq, d), np.float64)
    fp8 = k_cache.dtype == np.uint8
    for i in (range(b) if seqs is None else seqs):
        n = int(ctx_lens[i])
        k_seq = gather_seq(k_cache, block_tables[i], n)
        v_seq = gather_seq(v_cache, block_tables[i], n)
        if fp8:
            k_seq = dequant_kv(k_seq[None], k_scale, q_dtype)[0]
            v_seq = dequant_kv(v_seq[None], v_scale, q_dtype)[0]
        lo = max(0, n - 1 - window_left) if window_left >= 0 else 0
        out[i] = attend_one(q[i], k_seq[lo:], v_seq[lo:], scale, sinks)
    return out


def _prefill_one(qq: np.ndarray, ks: np.ndarray, vs: np.ndarray, scale: float,
                 causal: bool, window_left: int = -1, sinks: np.ndarray | None = None,
                 return_lse: bool = False):
    """_sdpa_one (attention_impl.py:606-622) in float64: qq [q_len, hq, d], ks [k_len,
    hk, d], vs [k_len, hk, dv] (dv may differ from d, as in MLA prefill); key_offset =
    k_len - q_len when causal, else all keys visible.  window_left >= 0 (causal): query
    j also drops keys before pos_j - window_left (triton_unified_attention.py:577-590);
    sinks as in attend_one.  return_lse: also the rows' log-sum-exp [hq, q_len],
    ln(sum over visible keys of e^(scale q.k)) plus e^sink with sinks (the denominator
    the output is divided by), -inf for a row with no visible key
    (flash_attn_varlen_func's return_softmax_lse, flash_attn_varlen.py:33-46)."""
    q_len, hq, _ = qq.shape
    k_len, hk, _ = ks.shape
    grp = hq // hk
    kh = np.repeat(ks.astype(np.float64), grp, axis=1)  # [k_len, hq, d]
    vh = np.repeat(vs.astype(np.float64), grp, axis=1)
    sc = np.einsum("jhd,thd->hjt", qq.astype(np.float64), kh) * scale  # [hq, q_len, k_len]
    pos = ((k_len - q_len) + np.arange(q_len)) if causal else np.full(q_len, k_len - 1)
    mask = np.arange(k_len)[None, :] <= pos[:, None]
    if window_left >= 0:
        mask &= np.arange(k_len)[None, :] >= pos[:, None] - window_left
    sc = np.where(mask[None], sc, -np.inf)
    m = sc.max(axis=-1, keepdims=True) if k_len else np.full((hq, q_len, 1), -np.inf)
    has = np.isfinite(m)
    if sinks is not None:  # the sink joins the max (only rows with a visible key matter)
        m = np.where(has, np.maximum(m, np.asarray(sinks, np.float64).reshape(hq, 1, 1)), m)
    e = np.where(has, np.exp(sc - np.where(has, m, 0.0)), 0.0)
    l = e.sum(-1, keepdims=True)
    if sinks is not None:
        l = np.where(l > 0, l + np.exp(np.asarray(sinks, np.float64).reshape(hq, 1, 1)
                                       - np.where(has, m, 0.0)), l)
    p = np.where(l > 0, e / np.where(l > 0, l, 1.0), 0.0)
    out = np.einsum("hjt,thd->jhd", p, vh)
    if not return_lse:
        return out
    with np.errstate(divide="ignore"):
        lse = np.where(l > 0, np.where(has, m, 0.0) + np.log(np.where(l > 0, l, 1.0)), -np.inf)
    return out, lse[..., 0]


def varlen_prefill(q: np.ndarray, key: np.ndarray, value: np.ndarray, cu_seqlens_q: np.ndarray,
                   cu_seqlens_k: np.ndarray, scale: float, causal: bool = True,
                   window_left: int = -1, sinks: np.ndarray | None = None,
                   return_lse: bool = False):
    """_prefill_torch_from_tensors (attention_impl.py:624-638): dense keys, sequence i's
    being rows cu_k[i]..cu_k[i+1] of key [total_k, hk, d] / value [total_k, hk, dv];
    the output is [total_q, hq, dv].  return_lse: also (out, lse [hq, total_q]), lse as
    in _prefill_one (FlashAttnVarlen's return_softmax_lse, flash_attn_varlen.py:33-46);
    rows of a sequence with no queries are not touched (-inf)."""
    total_q, hq, _ = q.shape
    out = np.zeros((total_q, hq, value.shape[-1]), np.float64)
    lse = np.full((hq, total_q), -np.inf)
    for i in range(len(cu_seqlens_q) - 1):
        qs, qe = int(cu_seqlens_q[i]), int(cu_seqlens_q[i + 1])
        ks, ke = int(cu_seqlens_k[i]), int(cu_seqlens_k[i + 1])
        if qe > qs:
            r = _prefill_one(q[qs:qe], key[ks:ke], value[ks:ke], scale, causal, window_left,
                             sinks, return_lse)
            if return_lse:
                out[qs:qe], lse[:, qs:qe] = r
            else:
                out[qs:qe] = r
    return (out, lse) if return_lse else out


def paged_prefill(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                  block_tables: np.ndarray, cu_seqlens_q: np.ndarray, cu_seqlens_k: np.ndarray,
                  scale: float, k_scale: np.ndarray | None = None,
                  v_scale: np.ndarray | None = None, q_dtype: str = "bf16",
                  causal: bool = True, window_left: int = -1,
                  sinks: np.ndarray | None = None, return_lse: bool = False):
    """_prefill_torch_from_cache + _sdpa_one (attention_impl.py:606-622, 640-652), the
    torch restatement of FlashAttnPrefill with a block table (flash_attn_prefill.py:28-74):
    sequence i's queries q[cu_q[i]:cu_q[i+1]] attend to the first k_len = cu_k[i+1]-cu_k[i]
    cached tokens, query j seeing keys [0, k_len - q_len + j] (key_offset = k_len - q_len).
    A query with no visible key gives a zero row.  float64 throughout.  The value cache
    may have its own head size (the output takes it); return_lse as varlen_prefill."""
    total_q, hq, _ = q.shape
    out = np.zeros((total_q, hq, v_cache.shape[-1]), np.float64)
    lse = np.full((hq, total_q), -np.inf)
    fp8 = k_cache.dtype == np.uint8
    for i in range(len(cu_seqlens_q) - 1):
        qs, qe = int(cu_seqlens_q[i]), int(cu_seqlens_q[i + 1])
        k_len = int(cu_seqlens_k[i + 1] - cu_seqlens_k[i])
        if qe == qs:
            continue
        ks = gather_seq(k_cache, block_tables[i], k_len)
        vs = gather_seq(v_cache, block_tables[i], k_len)
        if fp8:
            ks = dequant_kv(ks[None], k_scale, q_dtype)[0]
            vs = dequant_kv(vs[None], v_scale, q_dtype)[0]
        r = _prefill_one(q[qs:qe], ks, vs, scale, causal, window_left, sinks, return_lse)
        if return_lse:
            out[qs:qe], lse[:, qs:qe] = r
        else:
            out[qs:qe] = r
    return (out, lse) if return_lse else out


def attend_partials(q: np.ndarray, k_seq: np.ndarray, v_seq: np.ndarray, scale: float,
                    part_tokens: int):
    """Split-context partials of one sequence: per partition p the max m_p, the sum
    l_p = sum exp(s - m_p), and the unnormalised o_p = sum exp(s - m_p) v
    (the segment state of triton_unified_attention.py:815-1066)."""
    hq, d = q.shape
    n, hk, _ = k_seq.shape
    grp = hq // hk
    parts = []
    for t0 in range(0, n, part_tokens):
        ks, vs = k_seq[t0:t0 + part_tokens], v_seq[t0:t0 + part_tokens]
        qh = q.astype(np.float64).reshape(hk, grp, d)
        s = np.matmul(qh, ks.astype(np.float64).transpose(1, 2, 0)) * scale
        m = s.max(axis=-1)
        e = np.exp(s - m[..., None])
        parts.append((m.reshape(hq), e.sum(-1).reshape(hq),
                      np.matmul(e, vs.astype(np.float64).transpose(1, 0, 2)).reshape(hq, d)))
    return parts


def merge_partials(parts) -> np.ndarray:
    """Log-sum-exp merge of reduce_segments (triton_unified_attention.py:741-776):
    M = max m_p; L = sum l_p e^(m_p - M); O = sum o_p e^(m_p - M) / L; 0 if L == 0."""
    if not parts:
        return None
    m = np.stack([p[0] for p in parts])
    l = np.stack([p[1] for p in parts])
    o = np.stack([p[2] for p in parts])
    big_m = m.max(axis=0)
    f = np.exp(m - big_m)
    big_l = (l * f).sum(axis=0)
    acc = (o * f[..., None]).sum(axis=0)
    with np.errstate(invalid="ignore", divide="ignore"):
        res = np.where(big_l[..., None] == 0, 0.0, acc / big_l[..., None])
    return res


# ---------------------------------------------------------------------------
# merge_attn_states — fastkernels/tasks/baseline/L1/merge_attn_states.py:30-100,
# kernel merge_attn_states.cu:2443-2571
# ---------------------------------------------------------------------------


def merge_attn_states(prefix: np.ndarray, prefix_lse: np.ndarray, suffix: np.ndarray,
                      suffix_lse: np.ndarray, dtype: str,
                      prefill_tokens_with_context: int | None = None,
                      output_scale: float | None = None):
    """(out [T, H, D], out_lse [H, T]) of the two-partition LSE merge.

    output_scale (the fp8 output, USE_FP8_OUTPUT, cu:2436-2571): out holds e4m3fn codes
    (uint8) of every output value v -- the fp32 merge, not rounded to ``dtype``, or the
    copied prefix / suffix value -- as e4m3fn(fmax(-448, fmin(v * inv, 448))) with
    inv = 1 / output_scale in fp32 (so a NaN becomes 448, the IEEE fmin/fmax rule).

    Tokens t < P (P = prefill_tokens_with_context, default T): infinite lse read as
    -inf (cu:2476-2477); M = max(p, s); if M = -inf the prefix rows and -inf are
    emitted (cu:2489-2517); else weights e^(p-M)/E, e^(s-M)/E with E their sum,
    one rounding of the weighted sum to ``dtype`` (cu:2520-2565) and
    out_lse = log(E) + M (cu:2567-2571).  Tokens t >= P copy the suffix and its lse
    (cu:2443-2471)."""
    prefix = np.asarray(prefix, np.float32)
    suffix = np.asarray(suffix, np.float32)
    t_all = prefix.shape[0]
    n = t_all if prefill_tokens_with_context is None else min(int(prefill_tokens_with_context), t_all)
    out = suffix.copy()
    out_lse = np.asarray(suffix_lse, np.float32).copy()
    p = np.asarray(prefix_lse, np.float64)[:, :n].T  # [n, H]
    s = np.asarray(suffix_lse, np.float64)[:, :n].T
    p = np.where(np.isinf(p), -np.inf, p)
    s = np.where(np.isinf(s), -np.inf, s)
    m = np.maximum(p, s)
    empty = np.isneginf(m)
    mz = np.where(empty, 0.0, m)
    ep = np.where(empty, 0.0, np.exp(p - mz))
    es = np.where(empty, 0.0, np.exp(s - mz))
    e = np.where(empty, 1.0, ep + es)
    merged = prefix[:n].astype(np.float64) * (ep / e)[..., None] + \
        suffix[:n].astype(np.float64) * (es / e)[..., None]
    merged = merged.astype(np.float32)
    if output_scale is None:
        merged = round_to(merged, dtype)
    out[:n] = np.where(empty[..., None], prefix[:n], merged)
    out_lse[:, :n] = np.where(empty, -np.inf, np.log(e) + mz).T.astype(np.float32)
    if output_scale is not None:
        inv = np.float32(1.0) / np.float32(output_scale)
        x = out.astype(np.float32) * inv
        x = np.where(np.isnan(x), np.float32(E4M3FN_MAX), np.clip(x, -E4M3FN_MAX, E4M3FN_MAX))
        return fp8_e4m3fn_encode(x.astype(np.float32)), out_lse
    return out, out_lse


# ---------------------------------------------------------------------------
# SiLU-and-mul — SiluAndMul.forward_native, fastkernels/tasks/baseline/L1/silu_and_mul.py:19-22
# ---------------------------------------------------------------------------


def silu_and_mul(x: np.ndarray, dtype: str) -> np.ndarray:
    """cast(cast(silu(g)) * u) with g = x[..., :d], u = x[..., d:] (F.silu in the tensor
    dtype, then the product in the tensor dtype)."""
    x = np.asarray(x, np.float32)
    d = x.shape[-1] // 2
    g = x[..., :d].astype(np.float64)
    act = round_to((g / (1.0 + np.exp(-g))).astype(np.float32), dtype)
    return round_to(act * x[..., d:], dtype)


# ---------------------------------------------------------------------------
# Acceptance rule of the reference's bench: candidate output vs baseline output,
# fastkernels/bench.py:141-155 (tolerances), :172-178 (statuses), :1824-1896
# (_tensor_leaves, _compare_tensor, _compare)
# ---------------------------------------------------------------------------
PASSED = "PASSED"
INCORRECT_NUMERICAL = "INCORRECT_NUMERICAL"
INCORRECT_SHAPE = "INCORRECT_SHAPE"
INCORRECT_DTYPE = "INCORRECT_DTYPE"
SKIPPED = "SKIPPED"

REQUIRED_MATCHED_RATIO = 0.99
# (atol, rtol) by the reference tensor's dtype; fp8 outputs use (0.125, 0.125).
TOLERANCES = {"f32": (1e-5, 1e-3), "f64": (1e-5, 1e-3), "f16": (1e-2, 1e-2),
              "bf16": (1e-2, 1e-2), "fp8": (0.125, 0.125)}
DEFAULT_TOL = (1e-2, 1e-2)


def leaves(obj) -> list:
    """Array leaves of a nested tuple / list / dict (dict values in order); anything
    that is not an array (None, ints, strings) is dropped, as _tensor_leaves does."""
    if isinstance(obj, np.ndarray):
        return [obj]
    if isinstance(obj, (list, tuple)):
        return [t for x in obj for t in leaves(x)]
    if isinstance(obj, dict):
        return [t for v in obj.values() for t in leaves(v)]
    return []


def _norm32(x: np.ndarray) -> float:
    return float(np.sqrt(np.sum(np.square(x, dtype=np.float32), dtype=np.float32)))


def compare_tensor(out: np.ndarray, ref: np.ndarray, ref_dtype: str):
    """(ok, max_abs, max_rel, matched_ratio, detail) for one output, values compared in
    float32.  An element matches when |out - ref| <= atol + rtol * |ref| (and is
    finite); the output passes when at least REQUIRED_MATCHED_RATIO of its elements
    match.  NaN or Inf anywhere, or an all-zero output against a nonzero reference,
    fails outright."""
    atol, rtol = TOLERANCES.get(ref_dtype, DEFAULT_TOL)
    x = np.asarray(out, np.float32)
    y = np.asarray(ref, np.float32)
    inf = float("inf")
    if np.isnan(x).any() or np.isnan(y).any():
        return False, inf, inf, 0.0, "NaN in output"
    if np.isinf(x).any() or np.isinf(y).any():
        return False, inf, inf, 0.0, "Inf in output"
    ref_norm = _norm32(y)
    if ref_norm > 0 and _norm32(x) == 0:
        return False, ref_norm, ref_norm, 0.0, "output is all-zeros"
    if x.size == 0:
        return True, 0.0, 0.0, 1.0, ""
    abs_err = np.abs(x - y)
    max_abs = float(abs_err.max())
    exceed = (abs_err > atol + rtol * np.abs(y)) | ~np.isfinite(abs_err)
    matched = 1.0 - float(exceed.sum()) / exceed.size
    max_rel = float((abs_err / np.maximum(np.abs(y), np.float32(atol))).max())
    ok = matched >= REQUIRED_MATCHED_RATIO
    detail = "" if ok else f"only {matched:.4f} within atol={atol},rtol={rtol}"
    return ok, max_abs, max_rel, matched, detail


def compare(out, ref, ref_dtypes, out_dtypes=None, check_dtype: bool = True):
    """(status, max_abs, max_rel, matched_ratio, detail) for a candidate's outputs
    against the baseline's.  ``out`` and ``ref`` are arrays or nested tuples / lists /
    dicts of arrays (values); ``ref_dtypes`` / ``out_dtypes`` give each leaf's dtype
    tag (one tag for all leaves, or a list; ``out_dtypes`` defaults to ``ref_dtypes``).
    A reference whose nonempty leaves are all zero is SKIPPED (it cannot tell a
    stub from a kernel); otherwise leaves are compared in order and the first
    failing one decides."""
    o, r = leaves(out), leaves(ref)
    inf = float("inf")
    if len(o) != len(r):
        return INCORRECT_SHAPE, inf, inf, 0.0, f"output tensor count {len(o)} != {len(r)}"
    rd = [ref_dtypes] * len(r) if isinstance(ref_dtypes, str) else list(ref_dtypes)
    od = rd if out_dtypes is None else (
        [out_dtypes] * len(o) if isinstance(out_dtypes, str) else list(out_dtypes))
    nonempty = [x for x in r if x.size > 0]
    if nonempty and all(_norm32(np.asarray(x, np.float32)) == 0 for x in nonempty):
        return SKIPPED, 0.0, 0.0, 0.0, "skip: reference output is all-zeros"
    worst, max_abs, max_rel = 1.0, 0.0, 0.0
    for x, y, tx, ty in zip(o, r, od, rd):
        if tuple(x.shape) != tuple(y.shape):
            return INCORRECT_SHAPE, inf, inf, 0.0, f"shape {tuple(x.shape)} != {tuple(y.shape)}"
        if check_dtype and tx != ty:
            return INCORRECT_DTYPE, inf, inf, 0.0, f"dtype {tx} != {ty}"
        ok, a, rl, matched, detail = compare_tensor(x, y, ty)
        max_abs, max_rel = max(max_abs, a), max(max_rel, rl)
        worst = min(worst, matched)
        if not ok:
            return INCORRECT_NUMERICAL, max_abs, max_rel, worst, detail
    return PASSED, max_abs, max_rel, worst, ""
