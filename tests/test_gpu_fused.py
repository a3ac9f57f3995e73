"""GPU parity of the fused store + decode launch (fk_store_paged_decode).

The reference's decode step stores the new token's K/V (StoreKVCache) and then
runs the decode (FlashAttnDecode) (fastkernels/tasks/baseline/L2/
attention_impl.py:313-363).  The fused launch must leave the caches and the
output exactly as those two calls do (bit for bit: the kernel takes the new row
from registers instead of re-reading the cache), and the output must meet the
oracle's attention bar on the updated cache.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from fastkernels_amd import ops, workloads

pytestmark = pytest.mark.gpu


def _flush(msg):
    print(msg, flush=True)


def _plan(case, num_splits, max_seq_len=None):
    b, hq, d = case.q.shape
    hk = case.k_cache.shape[2]
    msl = case.max_seq_len if max_seq_len is None else max_seq_len
    part, nparts, nbytes = ops.paged_decode_plan(b, hq, hk, d, msl, num_splits)
    ws = torch.zeros(max(nbytes, 1), dtype=torch.uint8, device=case.q.device)
    return part, nparts, ws


def _separate(case, rows, num_splits, max_seq_len=None):
    """store_kvcache then paged_decode on private copies of the caches."""
    kc, vc = case.k_cache.clone(), case.v_cache.clone()
    ops.store_kvcache(rows.key, rows.value, kc, vc, rows.slot_mapping)
    part, nparts, ws = _plan(case, num_splits, max_seq_len)
    out = torch.full_like(case.q, float("nan"))
    ops.paged_decode(out, case.q, kc, vc, case.block_tables, case.ctx_lens, case.scale, part,
                     nparts, ws, case.k_scale, case.v_scale)
    torch.cuda.synchronize()
    return out, kc, vc


def _fused(case, rows, num_splits, max_seq_len=None, slot_mapping=None):
    kc, vc = case.k_cache.clone(), case.v_cache.clone()
    part, nparts, ws = _plan(case, num_splits, max_seq_len)
    out = torch.full_like(case.q, float("nan"))
    sm = rows.slot_mapping if slot_mapping is None else slot_mapping
    ops.store_paged_decode(out, case.q, rows.key, rows.value, kc, vc, sm, case.block_tables,
                           case.ctx_lens, case.scale, part, nparts, ws, case.k_scale,
                           case.v_scale)
    torch.cuda.synchronize()
    return out, kc, vc


def _assert_same(fused, sep, what):
    for name, a, b in zip(("out", "k_cache", "v_cache"), fused, sep):
        if a.dtype == torch.float8_e4m3fn:
            a, b = a.view(torch.uint8), b.view(torch.uint8)
        assert torch.equal(a, b), f"{what}: {name} differs from store_kvcache + paged_decode"


@pytest.mark.parametrize("num_splits", [0, 3, 64])
@pytest.mark.parametrize("slot_dtype", [torch.int64, torch.int32])
def test_fused_equals_store_then_decode_bf16(cuda, num_splits, slot_dtype):
    _flush(f"fused bf16 num_splits={num_splits} slots={slot_dtype}")
    case = workloads.c3_decode(cuda, batch=64, pool_blocks=1024, ctx_lo=1, ctx_hi=3000, seed=41)
    rows = workloads.decode_step_rows(case)
    rows.slot_mapping = rows.slot_mapping.to(slot_dtype)
    _assert_same(_fused(case, rows, num_splits), _separate(case, rows, num_splits),
                 f"bf16 splits={num_splits}")


@pytest.mark.parametrize("num_splits", [0, 16])
def test_fused_equals_store_then_decode_fp8(cuda, num_splits):
    _flush(f"fused fp8 num_splits={num_splits}")
    case = workloads.c5_fp8_decode(cuda, batch=8, ctx_lens=[5000, 1, 16, 17, 256, 257, 4096, 777],
                                   pool_blocks=64, seed=43)
    rows = workloads.decode_step_rows(case)
    _assert_same(_fused(case, rows, num_splits), _separate(case, rows, num_splits),
                 f"fp8 splits={num_splits}")


@pytest.mark.parametrize("block_size", [16, 64, 256])
def test_fused_edge_positions(cuda, block_size):
    """New token at the first/last row of a tile and of a page, ctx 1, empty
    sequences with slot -1, GQA 4/8."""
    lens = [1, 15, 16, 17, block_size - 1, block_size, block_size + 1, 0, 2 * block_size, 33, 0]
    for hq in (32, 64):
        _flush(f"fused edges bs={block_size} hq={hq}")
        case = workloads.c3_decode(cuda, num_heads=hq, block_size=block_size, pool_blocks=256,
                                   ctx_lens=lens, seed=44 + hq)
        rows = workloads.decode_step_rows(case)
        assert (rows.slot_mapping[torch.tensor(lens, device=cuda) == 0] == -1).all()
        for ns in (0, 2):
            _assert_same(_fused(case, rows, ns), _separate(case, rows, ns),
                         f"bs={block_size} hq={hq} splits={ns}")


def test_fused_orphan_slots_and_uncovered_positions(cuda):
    """Slots that are not position ctx-1 of their sequence (written by a designated
    work-group) and, with fixed partitions planned for a shorter max_seq_len, new
    tokens past the last partition: the caches still match store_kvcache, and so
    does the output (no sequence reads those slots here)."""
    case = workloads.c3_decode(cuda, batch=12, pool_blocks=200, ctx_lo=20, ctx_hi=2000, seed=46)
    rows = workloads.decode_step_rows(case)
    used = set(case.block_tables[case.block_tables >= 0].tolist())
    free = [p for p in range(200) if p not in used]
    sm = rows.slot_mapping.clone()
    bs = case.k_cache.shape[1]
    sm[3] = free[0] * bs + 5            # orphan in an unused page
    sm[7] = free[1] * bs + bs - 1
    sm[9] = 200 * bs + 3                 # out of range: skipped by both paths
    rows.slot_mapping = sm
    for ns, msl in ((0, None), (4, None), (2, 512)):
        _flush(f"fused orphans splits={ns} max_seq_len={msl}")
        _assert_same(_fused(case, rows, ns, msl), _separate(case, rows, ns, msl),
                     f"orphans splits={ns} msl={msl}")


def test_fused_against_oracle(cuda):
    """Output of the fused launch vs the oracle on the updated cache (bf16 bar)."""
    case = workloads.c3_decode(cuda, batch=16, pool_blocks=256, ctx_lo=1, ctx_hi=3000, seed=47)
    rows = workloads.decode_step_rows(case)
    out, kc, vc = _fused(case, rows, 0)
    bs = case.k_cache.shape[1]
    ctx = case.ctx_lens.cpu().numpy()
    bt = case.block_tables.cpu().numpy()
    q = case.q.float().cpu().numpy()
    got = out.float().cpu().numpy()
    for i in range(16):
        n = int(ctx[i])
        pages = (n + bs - 1) // bs
        ids = torch.from_numpy(bt[i, :pages].astype(np.int64)).to(cuda)
        kp, vp = kc[ids].float().cpu().numpy(), vc[ids].float().cpu().numpy()
        # the new token's row is in the cache at position n-1
        assert np.array_equal(kp.reshape(-1, *kp.shape[2:])[n - 1], rows.key[i].float().cpu().numpy())
        ref = oracle.paged_decode(q[i:i + 1], kp, vp, np.arange(pages)[None], np.array([n]),
                                  case.scale)[0]
        err = np.abs(got[i] - ref)
        assert (err <= 1e-2 + 1e-2 * np.abs(ref)).all(), f"seq {i}: max err {err.max()}"


def test_fused_candidate_forward_store(cuda):
    from fastkernels_amd.candidate.L1.flash_attn_decode import FlashAttnDecode
    from fastkernels_amd.candidate.L1.store_kvcache import StoreKVCache
    case = workloads.c3_decode(cuda, batch=24, pool_blocks=512, ctx_lo=1, ctx_hi=4000, seed=48)
    rows = workloads.decode_step_rows(case)
    attn = FlashAttnDecode(32, 8, 128, page_size=256)
    kc1, vc1 = case.k_cache.clone(), case.v_cache.clone()
    StoreKVCache()(rows.key, rows.value, kc1, vc1, rows.slot_mapping)
    ref = attn(case.q, kc1, vc1, cache_seqlens=case.ctx_lens, block_table=case.block_tables,
               softmax_scale=case.scale, causal=True, max_seq_len=4000)
    kc2, vc2 = case.k_cache.clone(), case.v_cache.clone()
    got = attn.forward_store(case.q, rows.key, rows.value, kc2, vc2, rows.slot_mapping,
                             cache_seqlens=case.ctx_lens, block_table=case.block_tables,
                             softmax_scale=case.scale, causal=True, max_seq_len=4000)
    torch.cuda.synchronize()
    assert torch.equal(got, ref) and torch.equal(kc1, kc2) and torch.equal(vc1, vc2)


# ---------------------------------------------------------------------------
# Fused per-head q/k RMSNorm + rotary + store_kvcache (fk_qk_norm_rope_store)
# ---------------------------------------------------------------------------
def _qkv_case(cuda, dtype, t, hq, hk, d, seed, pool_blocks=64, bs=16, max_pos=4096):
    g = torch.Generator().manual_seed(seed)
    qkv = (2 * torch.randn(t, (hq + 2 * hk) * d, generator=g)).to(dtype).to(cuda)
    positions = torch.randint(0, max_pos, (t,), generator=g).to(cuda)
    perm = torch.randperm(pool_blocks * bs, generator=g)[:t]
    slots = perm.to(torch.int64).to(cuda)
    kc = torch.randn(pool_blocks, bs, hk, d, generator=g).to(dtype).to(cuda)
    vc = torch.randn(pool_blocks, bs, hk, d, generator=g).to(dtype).to(cuda)
    qw = (1 + 0.2 * torch.randn(d, generator=g)).to(dtype).to(cuda)
    kw = (1 + 0.2 * torch.randn(d, generator=g)).to(dtype).to(cuda)
    return qkv, positions, slots, kc, vc, qw, kw


def _split(qkv, hq, hk, d):
    return qkv[:, :hq * d], qkv[:, hq * d:(hq + hk) * d], qkv[:, (hq + hk) * d:]


def _chain(qkv, positions, slots, kc, vc, qw, kw, eps, hq, hk, d, cache, neox):
    """rms_norm per head row, rotary_embedding, store_kvcache: the separate ops."""
    t = qkv.shape[0]
    q, k, v = _split(qkv, hq, hk, d)
    if qw is not None:
        for x, w, h in ((q, qw, hq), (k, kw, hk)):
            rows = x.reshape(t, h, d).contiguous()
            out = torch.empty_like(rows)
            ops.rms_norm(out, rows, w, eps)
            x.copy_(out.view(t, h * d))
    ops.rotary_embedding(positions, q, k, d, cache, neox)
    ops.store_kvcache(k.view(t, hk, d), v.view(t, hk, d), kc, vc, slots)


@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("norm", [True, False])
@pytest.mark.parametrize("cache_f32", [True, False])
def test_qk_norm_rope_store_equals_chain(cuda, neox, norm, cache_f32):
    """Qwen3-8B attention shapes (Hq 32, Hk 8, D 128), 256 tokens: bit-identical q, k
    and caches; tokens with slot -1 or an out-of-range position included."""
    from fastkernels_amd.candidate.L1.rotary_emb import RotaryEmbedding
    _flush(f"qk_norm_rope_store neox={neox} norm={norm} cache_f32={cache_f32}")
    t, hq, hk, d = 256, 32, 8, 128
    qkv, pos, slots, kc, vc, qw, kw = _qkv_case(cuda, torch.bfloat16, t, hq, hk, d, seed=61)
    pos[3] = -1
    pos[10] = 4096  # == max_position: not rotated
    slots[5] = -1
    slots[6] = kc.shape[0] * kc.shape[1]  # out of range: not stored
    rope = RotaryEmbedding(d, 4096, 1e6, is_neox_style=neox).to(cuda)
    cache = rope.cos_sin_cache if cache_f32 else rope.cos_sin_cache.bfloat16()
    eps = 1e-6
    a = (qkv.clone(), kc.clone(), vc.clone())
    _chain(a[0], pos, slots, a[1], a[2], qw if norm else None, kw, eps, hq, hk, d, cache, neox)
    b = (qkv.clone(), kc.clone(), vc.clone())
    q, k, v = _split(b[0], hq, hk, d)
    ops.qk_norm_rope_store(pos, q, k, v, b[1], b[2], slots, d, cache, neox,
                           qw if norm else None, kw if norm else None, eps)
    torch.cuda.synchronize()
    for name, x, y in zip(("qkv", "k_cache", "v_cache"), a, b):
        assert torch.equal(x, y), f"{name} differs from rms_norm + rotary + store_kvcache"


def test_qk_norm_rope_store_against_oracle(cuda):
    """The fused result against the oracle's rms_norm -> rotary -> store on the same
    inputs (bf16 bar), and v copied bit-exactly."""
    t, hq, hk, d = 64, 16, 4, 128
    qkv, pos, slots, kc, vc, qw, kw = _qkv_case(cuda, torch.bfloat16, t, hq, hk, d, seed=62)
    cs = oracle.rope_cos_sin_cache(d, 4096, 1e6)
    cache = torch.from_numpy(cs).to(cuda)
    x = qkv.float().cpu().numpy()
    q0, k0, v0 = x[:, :hq * d], x[:, hq * d:(hq + hk) * d], x[:, (hq + hk) * d:]
    qn = oracle.rms_norm(q0.reshape(t, hq, d), qw.float().cpu().numpy(), 1e-6, "bf16")
    kn = oracle.rms_norm(k0.reshape(t, hk, d), kw.float().cpu().numpy(), 1e-6, "bf16")
    qr, kr = oracle.rotary(pos.cpu().numpy(), qn.reshape(t, -1), kn.reshape(t, -1), d, cs, True,
                           "bf16")
    q, k, v = _split(qkv, hq, hk, d)
    ops.qk_norm_rope_store(pos, q, k, v, kc, vc, slots, d, cache, True, qw, kw, 1e-6)
    torch.cuda.synchronize()
    for got, ref, nm in ((q, qr, "q"), (k, kr, "k")):
        g = got.float().cpu().numpy()
        err = np.abs(g - ref)
        assert (err <= 1e-2 + 1e-2 * np.abs(ref)).all(), f"{nm}: max err {err.max()}"
    kflat = kc.view(-1, hk * d)
    vflat = vc.view(-1, hk * d)
    assert torch.equal(kflat[slots], k) and torch.equal(vflat[slots], v)


@pytest.mark.parametrize("dtype,d,rot", [(torch.float32, 128, 128), (torch.float32, 64, 64),
                                         (torch.bfloat16, 128, 64), (torch.float16, 256, 256)])
def test_qk_norm_rope_store_dtypes_and_partial_rotary(cuda, dtype, d, rot):
    _flush(f"qk_norm_rope_store {dtype} d={d} rot={rot}")
    t, hq, hk = 33, 8, 2
    qkv, pos, slots, kc, vc, qw, kw = _qkv_case(cuda, dtype, t, hq, hk, d, seed=63)
    slots = slots.to(torch.int32)
    inv = 1.0 / (1e4 ** (torch.arange(0, rot, 2, dtype=torch.float32) / rot))
    ang = torch.outer(torch.arange(4096, dtype=torch.float32), inv)
    cache = torch.cat((ang.cos(), ang.sin()), -1).to(cuda)
    for neox in (True, False):
        a = (qkv.clone(), kc.clone(), vc.clone())
        _chain(a[0], pos, slots, a[1], a[2], qw, kw, 1e-5, hq, hk, d, cache, neox)
        b = (qkv.clone(), kc.clone(), vc.clone())
        q, k, v = _split(b[0], hq, hk, d)
        ops.qk_norm_rope_store(pos, q, k, v, b[1], b[2], slots, d, cache, neox, qw, kw, 1e-5)
        torch.cuda.synchronize()
        for name, x, y in zip(("qkv", "k_cache", "v_cache"), a, b):
            assert torch.equal(x, y), f"{name} differs (neox={neox})"


def test_qk_norm_rope_store_candidate(cuda):
    """RotaryEmbedding.forward_store with RMSNorm q/k norms == the modules one by one
    (the reference's Qwen3 path: norms on [N, H, D] views, rotary, StoreKVCache)."""
    from fastkernels_amd.candidate.L1.rms_norm import RMSNorm
    from fastkernels_amd.candidate.L1.rotary_emb import RotaryEmbedding
    from fastkernels_amd.candidate.L1.store_kvcache import StoreKVCache
    t, hq, hk, d = 48, 32, 8, 128
    qkv, pos, slots, kc, vc, qw, kw = _qkv_case(cuda, torch.bfloat16, t, hq, hk, d, seed=64)
    qn, kn = RMSNorm(d, eps=1e-6), RMSNorm(d, eps=1e-6)
    qn.weight.data.copy_(qw.float())
    kn.weight.data.copy_(kw.float())
    qn, kn = qn.to(cuda).to(torch.bfloat16), kn.to(cuda).to(torch.bfloat16)
    rope = RotaryEmbedding(d, 4096, 1e6).to(cuda)
    # module by module, as attention.py:120-140 and attention_impl.py:323-325
    a = qkv.clone()
    q, k, v = _split(a, hq, hk, d)
    q2 = qn(q.view(t, hq, d)).view(t, hq * d)
    k2 = kn(k.view(t, hk, d)).view(t, hk * d)
    q2, k2 = rope(pos, q2, k2)
    kc1, vc1 = kc.clone(), vc.clone()
    StoreKVCache()(k2.view(t, hk, d), v.view(t, hk, d), kc1, vc1, slots)
    # fused
    b = qkv.clone()
    qb, kb, vb = _split(b, hq, hk, d)
    kc2, vc2 = kc.clone(), vc.clone()
    rope.forward_store(pos, qb, kb, vb, kc2, vc2, slots, q_norm=qn, k_norm=kn)
    torch.cuda.synchronize()
    assert torch.equal(qb, q2) and torch.equal(kb, k2)
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2)


def test_fused_paths_with_fp8_cache_and_bf16_rows(cuda):
    """bf16 new rows into an fp8 cache: forward_store (decode) and forward_store
    (rotary) fall back to the converting store; results equal the module chain."""
    from fastkernels_amd.candidate.L1.flash_attn_decode import FlashAttnDecode
    from fastkernels_amd.candidate.L1.rotary_emb import RotaryEmbedding
    from fastkernels_amd.candidate.L1.store_kvcache import StoreKVCache
    case = workloads.c5_fp8_decode(cuda, batch=4, ctx_lens=[100, 1, 300, 17], pool_blocks=8,
                                   seed=49)
    rows = workloads.decode_step_rows(case)
    kb, vb = rows.key.float().bfloat16(), rows.value.float().bfloat16()  # bf16 rows
    attn = FlashAttnDecode(64, 8, 128, page_size=256)
    kw = dict(cache_seqlens=case.ctx_lens, block_table=case.block_tables, softmax_scale=case.scale,
              k_scale=case.k_scale, v_scale=case.v_scale, max_seq_len=300)
    kc1, vc1 = case.k_cache.clone(), case.v_cache.clone()
    StoreKVCache()(kb, vb, kc1, vc1, rows.slot_mapping)
    ref = attn(case.q, kc1, vc1, **kw)
    kc2, vc2 = case.k_cache.clone(), case.v_cache.clone()
    got = attn.forward_store(case.q, kb, vb, kc2, vc2, rows.slot_mapping, **kw)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    assert torch.equal(kc1.view(torch.uint8), kc2.view(torch.uint8))
    # rotary + store into the fp8 cache
    t = 4
    qkv = torch.randn(t, (64 + 16) * 128, device=cuda).bfloat16()
    pos = torch.tensor([3, 7, 100, 2000], device=cuda)
    rope = RotaryEmbedding(128, 4096, 1e6).to(cuda)
    a = qkv.clone()
    qa, ka, va = a[:, :64 * 128], a[:, 64 * 128:72 * 128], a[:, 72 * 128:]
    kc3, vc3 = case.k_cache.clone(), case.v_cache.clone()
    rope(pos, qa, ka)
    StoreKVCache()(ka.view(t, 8, 128), va.view(t, 8, 128), kc3, vc3, rows.slot_mapping)
    b = qkv.clone()
    qb, kb2, vb2 = b[:, :64 * 128], b[:, 64 * 128:72 * 128], b[:, 72 * 128:]
    kc4, vc4 = case.k_cache.clone(), case.v_cache.clone()
    rope.forward_store(pos, qb, kb2, vb2, kc4, vc4, rows.slot_mapping)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert torch.equal(kc3.view(torch.uint8), kc4.view(torch.uint8))
    assert torch.equal(vc3.view(torch.uint8), vc4.view(torch.uint8))
