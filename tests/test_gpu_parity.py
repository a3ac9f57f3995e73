"""GPU parity: the gfx950 kernels (through the C ABI) against the CPU oracle.

Bars: store_kvcache bit-exact; bf16 ops within atol=rtol=1e-2 of the oracle's
fp32-upcast result (every element, stricter than the reference harness's 99%
rule, fastkernels/bench.py:142-155); fp8-KV attention within atol=rtol=3e-2;
fp32 outputs within the harness's fp32 tolerance (atol 1e-5, rtol 1e-3).
Sizes are the benchmark configurations (C1-C5) where the oracle finishes in
seconds, and small edge cases otherwise.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from fastkernels_amd import ops, workloads
from oracle.harness import fix_paged_decode

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2
FP8_TOL = 3e-2


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def assert_close(got, ref, atol, rtol, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} != {ref.shape}"
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    if bad.any():
        i = np.unravel_index(np.argmax(err - (atol + rtol * np.abs(ref))), err.shape)
        raise AssertionError(f"{what}: {int(bad.sum())}/{bad.size} outside atol={atol} rtol={rtol};"
                             f" worst at {i}: got {got[i]} ref {ref[i]}; max abs {err.max():.3g}")


def _flush(msg):
    print(msg, flush=True)


# ---------------------------------------------------------------------------
# store_kvcache (bit-exact)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("slot_dtype", [torch.int64, torch.int32])
def test_store_kvcache_c2_bitexact(cuda, slot_dtype):
    _flush(f"store_kvcache C2 slot_dtype={slot_dtype}")
    c = workloads.c2_store(cuda, slot_dtype=slot_dtype)
    ops.store_kvcache(c.key, c.value, c.k_cache, c.v_cache, c.slot_mapping)
    torch.cuda.synchronize()
    as_u16 = lambda t: t.view(torch.int16).cpu().numpy()
    kc0 = np.zeros(c.k_cache.shape, np.int16)
    ek, ev = oracle.store_kvcache(as_u16(c.key), as_u16(c.value), kc0, kc0,
                                  c.slot_mapping.cpu().numpy())
    assert np.array_equal(as_u16(c.k_cache), ek)
    assert np.array_equal(as_u16(c.v_cache), ev)


def test_store_kvcache_strided_views_and_edges(cuda):
    """key/value as strided views of a fused qkv row (attention_impl.py:319-325),
    slots -1 and past the cache end skipped, empty input, int32 slots."""
    g = torch.Generator().manual_seed(7)
    n, hq, hk, d, nb, bs = 37, 4, 2, 128, 8, 16
    qkv = torch.randn(n, (hq + 2 * hk) * d, generator=g).to(torch.bfloat16).to(cuda)
    k = qkv[:, hq * d:(hq + hk) * d].view(n, hk, d)
    v = qkv[:, (hq + hk) * d:].view(n, hk, d)
    slots = torch.randperm(nb * bs, generator=g)[:n]
    slots[::5] = -1
    slots[3] = nb * bs + 11  # past the end: must be skipped, not written
    kc = torch.zeros(nb, bs, hk, d, dtype=torch.bfloat16, device=cuda)
    vc = torch.zeros_like(kc)
    ops.store_kvcache(k, v, kc, vc, slots.to(torch.int32).to(cuda))
    ops.store_kvcache(k[:0], v[:0], kc, vc, slots[:0].to(cuda))
    torch.cuda.synchronize()
    u16 = lambda t: t.contiguous().view(torch.int16).cpu().numpy()
    sl = slots.numpy().copy()
    sl[sl >= nb * bs] = -1
    ek, ev = oracle.store_kvcache(u16(k), u16(v), np.zeros(kc.shape, np.int16),
                                  np.zeros(kc.shape, np.int16), sl)
    assert np.array_equal(u16(kc), ek) and np.array_equal(u16(vc), ev)


@pytest.mark.parametrize("dtype,hk,d", [(torch.float8_e4m3fn, 8, 128), (torch.float32, 2, 64),
                                        (torch.bfloat16, 3, 5)])
def test_store_kvcache_dtypes(cuda, dtype, hk, d):
    g = torch.Generator().manual_seed(11)
    n, nb, bs = 50, 4, 32
    key = torch.randn(n, hk, d, generator=g).to(dtype).to(cuda)
    val = torch.randn(n, hk, d, generator=g).to(dtype).to(cuda)
    slots = torch.randperm(nb * bs, generator=g)[:n].to(cuda)
    kc = torch.zeros(nb, bs, hk, d, dtype=dtype, device=cuda)
    vc = torch.zeros_like(kc)
    ops.store_kvcache(key, val, kc, vc, slots)
    torch.cuda.synchronize()
    iv = torch.int8 if dtype.itemsize == 1 else (torch.int16 if dtype.itemsize == 2 else torch.int32)
    raw = lambda t: t.view(iv).cpu().numpy()
    ek, ev = oracle.store_kvcache(raw(key), raw(val), np.zeros(kc.shape, raw(kc).dtype),
                                  np.zeros(kc.shape, raw(kc).dtype), slots.cpu().numpy())
    assert np.array_equal(raw(kc), ek) and np.array_equal(raw(vc), ev)


@pytest.mark.parametrize("dtype,hk,d,page", [(torch.bfloat16, 8, 128, 16), (torch.bfloat16, 8, 128, 64),
                                             (torch.float8_e4m3fn, 4, 128, 32),
                                             (torch.float32, 2, 64, 16), (torch.bfloat16, 3, 5, 8)])
@pytest.mark.parametrize("slot_dtype", [torch.int64, torch.int32])
def test_store_kvcache_hnd_bitexact(cuda, dtype, hk, d, page, slot_dtype):
    """StoreKVCacheHND (store_kvcache.py:85-99): HND caches [num_blocks, Hk, page, D],
    key/value as strided views of a fused qkv row, slots -1 and past the end skipped;
    the 16-byte path and the element path (D = 5)."""
    from fastkernels_amd.candidate.L1.store_kvcache import StoreKVCacheHND

    g = torch.Generator().manual_seed(13 + d + page)
    n, nb, hq = 300, 40, 2 * hk
    qkv = torch.randn(n, (hq + 2 * hk) * d, generator=g).to(dtype).to(cuda)
    k = qkv[:, hq * d:(hq + hk) * d].view(n, hk, d)
    v = qkv[:, (hq + hk) * d:].view(n, hk, d)
    slots = torch.randperm(nb * page, generator=g)[:n] if n <= nb * page else None
    if slots is None:
        pytest.skip("cache too small for distinct slots")
    slots[::7] = -1
    slots[5] = nb * page + 2
    kc = torch.zeros(nb, hk, page, d, dtype=dtype, device=cuda)
    vc = torch.zeros_like(kc)
    StoreKVCacheHND(page)(k, v, kc, vc, slots.to(slot_dtype).to(cuda))
    torch.cuda.synchronize()
    iv = {1: torch.int8, 2: torch.int16, 4: torch.int32}[kc.element_size()]
    raw = lambda t: t.contiguous().view(iv).cpu().numpy()  # noqa: E731
    z = np.zeros(kc.shape, raw(kc).dtype)
    ek, ev = oracle.store_kvcache_hnd(raw(k), raw(v), z, z, slots.numpy(), page)
    assert np.array_equal(raw(kc), ek) and np.array_equal(raw(vc), ev)


def test_gemma4_proportional_rotary(cuda):
    """Gemma4ProportionalRotaryEmbedding: base-class forward over the whole head with the
    proportional cache (identity pairs past rotary_dim), against the oracle's NeoX
    rotation with the same cache."""
    from fastkernels_amd.candidate.L1.rotary_emb import Gemma4ProportionalRotaryEmbedding

    g = torch.Generator().manual_seed(17)
    t, hq, hk, d = 64, 8, 2, 256
    rope = Gemma4ProportionalRotaryEmbedding(d, 64, 4096, 1e6).to(cuda)
    qkv = torch.randn(t, (hq + 2 * hk) * d, generator=g).to(torch.bfloat16).to(cuda)
    q, k = qkv[:, :hq * d], qkv[:, hq * d:(hq + hk) * d]
    pos = torch.randint(0, 4096, (t,), generator=g).to(cuda)
    q0, k0 = f32(q), f32(k)
    rope(pos, q, k)
    torch.cuda.synchronize()
    rq, rk = oracle.rotary(pos.cpu().numpy(), q0, k0, d, f32(rope.cos_sin_cache), True, "bf16")
    assert_close(f32(q), rq, BF16_TOL, BF16_TOL, "q")
    assert_close(f32(k), rk, BF16_TOL, BF16_TOL, "k")
    # the identity pairs (dims 32..127 and 160..255 of each head) are untouched
    qh, q0h = f32(q).reshape(t, hq, d), q0.reshape(t, hq, d)
    assert np.array_equal(qh[..., 32:128], q0h[..., 32:128])
    assert np.array_equal(qh[..., 160:], q0h[..., 160:])


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------
_DT = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("hidden", [1024, 4096])
def test_fused_add_rmsnorm(cuda, dtype, hidden):
    _flush(f"fused_add_rmsnorm {dtype} H={hidden}")
    c = workloads.c1_norm(cuda, dtype=dtype, hidden=hidden)
    x0, r0 = f32(c.x), f32(c.residual)
    ref_out, ref_res = oracle.rms_norm(x0, f32(c.weight), c.eps, _DT[dtype], residual=r0)
    x, r = c.x.clone(), c.residual.clone()
    ops.fused_add_rms_norm(x, r, c.weight, c.eps)
    torch.cuda.synchronize()
    assert np.array_equal(f32(r), ref_res), "new residual must be bit-exact cast(x + r)"
    tol = BF16_TOL if dtype != torch.float32 else 1e-5
    assert_close(f32(x), ref_out, tol, tol if dtype != torch.float32 else 1e-3, "out")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("hidden", [64, 1024, 5120, 1001, 16384])
def test_rmsnorm_plain(cuda, dtype, hidden):
    c = workloads.c1_norm(cuda, dtype=dtype, tokens=33, hidden=hidden)
    out = torch.empty_like(c.x)
    ops.rms_norm(out, c.x, c.weight, c.eps)
    torch.cuda.synchronize()
    ref = oracle.rms_norm(f32(c.x), f32(c.weight), c.eps, _DT[dtype])
    tol = (BF16_TOL, BF16_TOL) if dtype != torch.float32 else (1e-5, 1e-3)
    assert_close(f32(out), ref, *tol, f"rmsnorm H={hidden}")


def test_rmsnorm_strided_rows(cuda):
    g = torch.Generator().manual_seed(3)
    big = torch.randn(40, 3 * 512, generator=g).to(torch.bfloat16).to(cuda)
    x = big[:, 512:1024]  # row stride 1536
    res = torch.randn(40, 512, generator=g).to(torch.bfloat16).to(cuda)
    w = (1 + 0.1 * torch.randn(512, generator=g)).to(torch.bfloat16).to(cuda)
    ref_out, ref_res = oracle.rms_norm(f32(x), f32(w), 1e-6, "bf16", residual=f32(res))
    before = big.clone()
    ops.fused_add_rms_norm(x, res, w, 1e-6)
    torch.cuda.synchronize()
    assert np.array_equal(f32(res), ref_res)
    assert_close(f32(x), ref_out, BF16_TOL, BF16_TOL)
    assert torch.equal(big[:, :512], before[:, :512]) and torch.equal(big[:, 1024:], before[:, 1024:])


# ---------------------------------------------------------------------------
# Rotary
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("is_neox", [True, False])
@pytest.mark.parametrize("cache_dtype", [torch.float32, torch.bfloat16])
def test_rotary_c4(cuda, is_neox, cache_dtype):
    """C4 dims: q [256, 32*128], k [256, 8*128] as strided views of qkv, theta 1e6."""
    _flush(f"rotary neox={is_neox} cache={cache_dtype}")
    t, hq, hk, d = 256, 32, 8, 128
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn(t, (hq + 2 * hk) * d, generator=g).to(torch.bfloat16).to(cuda)
    pos = torch.randint(0, 8192, (t,), generator=g).to(cuda)
    cs_np = oracle.rope_cos_sin_cache(d, 8192, 1e6)
    cache = torch.from_numpy(cs_np).to(cuda).to(cache_dtype)
    q = qkv[:, :hq * d]
    k = qkv[:, hq * d:(hq + hk) * d]
    q0, k0, v0 = f32(q), f32(k), qkv[:, (hq + hk) * d:].clone()
    ref_q, ref_k = oracle.rotary(pos.cpu().numpy(), q0, k0, d, f32(cache), is_neox, "bf16")
    ops.rotary_embedding(pos, q, k, d, cache, is_neox)
    torch.cuda.synchronize()
    assert_close(f32(q), ref_q, BF16_TOL, BF16_TOL, "q")
    assert_close(f32(k), ref_k, BF16_TOL, BF16_TOL, "k")
    assert torch.equal(qkv[:, (hq + hk) * d:], v0), "v slice must be untouched"


def test_rotary_partial_and_f32(cuda):
    """rot_dim < head_size (scalar path), fp32 tensors, key=None, out-of-range position."""
    t, h, d, rot = 9, 3, 64, 32
    g = torch.Generator().manual_seed(9)
    q = torch.randn(t, h * d, generator=g).to(cuda)
    pos = torch.randint(0, 100, (t,), generator=g)
    pos[4] = 100  # out of range: token left unchanged
    cs = oracle.rope_cos_sin_cache(rot, 100, 1e4)
    q0 = f32(q)
    ref_q, _ = oracle.rotary(np.clip(pos.numpy(), 0, 99), q0, None, d, cs, True, "f32")
    ref_q[4] = q0[4]
    ops.rotary_embedding(pos.to(cuda), q, None, d, torch.from_numpy(cs).to(cuda), True)
    torch.cuda.synchronize()
    assert_close(f32(q), ref_q, 1e-5, 1e-4)


# ---------------------------------------------------------------------------
# SiLU-and-mul
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype,shape", [(torch.bfloat16, (256, 2 * 12288)),
                                         (torch.bfloat16, (7, 2 * 1003)),
                                         (torch.float16, (16, 2 * 4096)),
                                         (torch.float32, (5, 2 * 512))])
def test_silu_and_mul(cuda, dtype, shape):
    g = torch.Generator().manual_seed(13)
    x = (3 * torch.randn(*shape, generator=g)).to(dtype).to(cuda)
    out = torch.empty(shape[0], shape[1] // 2, dtype=dtype, device=cuda)
    ops.silu_and_mul(out, x)
    torch.cuda.synchronize()
    ref = oracle.silu_and_mul(f32(x), _DT[dtype])
    tol = (BF16_TOL, BF16_TOL) if dtype != torch.float32 else (1e-5, 1e-4)
    assert_close(f32(out), ref, *tol)


@pytest.mark.parametrize("rows,d", [(70000, 256), (65536, 8), (70001, 12)])
def test_silu_and_mul_many_rows(cuda, rows, d):
    """More rows than a grid's y dimension holds (65,535): a long prefill chunk through
    SiluAndMul (the reference accepts any token count, silu_and_mul.py:24-30).  d = 12 is
    not a multiple of the 8-element vector, so it takes the scalar kernel."""
    _flush(f"silu_and_mul rows={rows} d={d}")
    g = torch.Generator().manual_seed(rows)
    x = (3 * torch.randn(rows, 2 * d, generator=g)).to(torch.bfloat16).to(cuda)
    out = torch.full((rows, d), float("nan"), dtype=torch.bfloat16, device=cuda)
    ops.silu_and_mul(out, x)
    torch.cuda.synchronize()
    assert_close(f32(out), oracle.silu_and_mul(f32(x), "bf16"), BF16_TOL, BF16_TOL,
                 f"silu rows={rows}")


# ---------------------------------------------------------------------------
# Paged decode attention
# ---------------------------------------------------------------------------
def run_decode(case, num_splits=0, max_seq_len=None):
    b, hq, d = case.q.shape
    hk = case.k_cache.shape[2]
    msl = case.max_seq_len if max_seq_len is None else max_seq_len
    part, nparts, nbytes = ops.paged_decode_plan(b, hq, hk, d, msl, num_splits)
    ws = torch.zeros(max(nbytes, 1), dtype=torch.uint8, device=case.q.device)
    out = torch.full_like(case.q, float("nan"))
    ops.paged_decode(out, case.q, case.k_cache, case.v_cache, case.block_tables, case.ctx_lens,
                     case.scale, part, nparts, ws, case.k_scale, case.v_scale)
    torch.cuda.synchronize()
    return out


def oracle_decode(case, seqs=None, window_left=-1, sinks=None):
    """Oracle on the pages the selected sequences use (host copies of those pages only)."""
    b = case.q.shape[0]
    seqs = list(range(b)) if seqs is None else list(seqs)
    bs = case.k_cache.shape[1]
    ctx = case.ctx_lens.cpu().numpy()
    bt = case.block_tables.cpu().numpy()
    fp8 = case.k_cache.dtype == torch.float8_e4m3fn
    out = np.zeros(tuple(case.q.shape), np.float64)
    q = f32(case.q)
    for i in seqs:
        n = int(ctx[i])
        pages = (n + bs - 1) // bs
        ids = torch.from_numpy(bt[i, :pages].astype(np.int64)).to(case.k_cache.device)
        if fp8:
            kp = case.k_cache[ids].view(torch.uint8).cpu().numpy()
            vp = case.v_cache[ids].view(torch.uint8).cpu().numpy()
        else:
            kp = f32(case.k_cache[ids])
            vp = f32(case.v_cache[ids])
        local_bt = np.arange(pages)[None]
        ks = None if case.k_scale is None else case.k_scale.cpu().numpy()
        vs = None if case.v_scale is None else case.v_scale.cpu().numpy()
        out[i] = oracle.paged_decode(q[i:i + 1], kp, vp, local_bt, np.array([n]), case.scale,
                                     ks, vs, window_left=window_left,
                                     sinks=None if sinks is None else f32(sinks))[0]
    return out


@pytest.mark.parametrize("block_size", [256, 64, 16])
def test_paged_decode_c3_north_star(cuda, block_size):
    """Full C3 launch (64 seqs, ctx U[512, 8192]); every sequence against the oracle.
    Also at 16-token pages (what the reference engine's AttnBackendConfig.auto_detect
    picks on this GPU, infra/context.py:68-73) and 64, over a pool of the same bytes."""
    _flush(f"paged_decode C3, block_size {block_size}")
    case = workloads.c3_decode(cuda, block_size=block_size, pool_blocks=4096 * 256 // block_size)
    out = run_decode(case)
    ref = oracle_decode(case)
    got = f32(out)
    assert np.isfinite(got).all()
    assert_close(got, ref, BF16_TOL, BF16_TOL, "C3")


@pytest.mark.parametrize("num_splits", [0, 1, 3, 16, 64])
def test_paged_decode_split_invariance(cuda, num_splits):
    """Any partition count gives the unsplit result (the LSE merge is exact)."""
    case = workloads.c3_decode(cuda, batch=6, num_heads=8, kv_heads=2, pool_blocks=64,
                               ctx_lo=1, ctx_hi=2000, seed=21)
    ref = oracle_decode(case)
    assert_close(f32(run_decode(case, num_splits)), ref, BF16_TOL, BF16_TOL, f"splits={num_splits}")


@pytest.mark.parametrize("num_splits", [1, 3, 16])
def test_paged_decode_fixed_partitions_past_max_seq_len(cuda, num_splits):
    """A fixed-partition plan made for a max_seq_len below the real contexts (a graph
    replayed after the contexts grew): the last partition runs on to the context end,
    so no key is dropped."""
    case = workloads.c3_decode(cuda, batch=5, num_heads=16, kv_heads=4, pool_blocks=96,
                               ctx_lo=900, ctx_hi=4000, seed=23)
    ref = oracle_decode(case)
    out = run_decode(case, num_splits, max_seq_len=700)
    assert_close(f32(out), ref, BF16_TOL, BF16_TOL, f"splits={num_splits}, max_seq_len 700")


@pytest.mark.parametrize("hq,hk", [(8, 8), (16, 8), (32, 8), (64, 8), (16, 1), (32, 2)])
@pytest.mark.parametrize("block_size", [16, 64, 256])
def test_paged_decode_gqa_blocks(cuda, hq, hk, block_size):
    ctx = [1, 15, 16, 17, 255, 256, 257, 1000]
    pool = sum((n + block_size - 1) // block_size for n in ctx) + 5
    case = workloads.c3_decode(cuda, num_heads=hq, kv_heads=hk, block_size=block_size,
                               pool_blocks=pool, ctx_lens=ctx, seed=31 + hq + block_size)
    assert_close(f32(run_decode(case)), oracle_decode(case), BF16_TOL, BF16_TOL,
                 f"hq={hq} hk={hk} bs={block_size}")


@pytest.mark.parametrize("lens", [
    [100_000],                                  # one sequence cut across every work-group
    [0, 1, 17, 0, 33, 0, 0, 5, 4096, 0, 16],    # empties between cut and whole sequences
    "many",                                     # 300 short sequences: more than work-groups
])
def test_paged_decode_balanced_schedule(cuda, lens):
    """The length-balanced schedule: sequences finished in place, cut across ranges,
    and empty, against the oracle; and equal to the fixed-partition schedule."""
    if lens == "many":
        lens = np.random.default_rng(71).integers(0, 100, 300).tolist()
    bs = 16
    pool = sum((n + bs - 1) // bs for n in lens) + 3
    case = workloads.c3_decode(cuda, num_heads=8, kv_heads=2, block_size=bs, pool_blocks=pool,
                               ctx_lens=lens, seed=81)
    seqs = [i for i in range(len(lens))][:64]
    got = f32(run_decode(case, 0))
    assert_close(got[seqs], oracle_decode(case, seqs)[seqs], BF16_TOL, BF16_TOL, "balanced")
    assert_close(got, f32(run_decode(case, 4)), BF16_TOL, BF16_TOL, "balanced vs fixed")
    for i, n in enumerate(lens):
        if n == 0:
            assert not got[i].any()


def test_paged_decode_batch_above_balanced_limit(cuda):
    """More than 8192 sequences: the plan falls back to fixed partitions (the balanced
    schedule keeps its tile prefix sums in LDS); every row against the oracle, empty
    sequences zero, with and without a window and sinks."""
    _flush("decode batch 9000 (fixed-partition fallback)")
    rng = np.random.default_rng(97)
    lens = rng.integers(0, 40, 9000).tolist()
    bs = 16
    pool = sum((n + bs - 1) // bs for n in lens) + 2
    case = workloads.c3_decode(cuda, num_heads=8, kv_heads=2, block_size=bs, pool_blocks=pool,
                               ctx_lens=lens, seed=98)
    plan = ops.paged_decode_plan(9000, 8, 2, 128, case.max_seq_len, 0)
    assert plan.part_tokens > 0  # fixed partitions
    seqs = list(range(0, 9000, 37))
    got = f32(run_decode_ws(case))
    assert_close(got[seqs], oracle_decode(case, seqs)[seqs], BF16_TOL, BF16_TOL, "batch 9000")
    for i, n in enumerate(lens):
        if n == 0:
            assert not got[i].any()
    g = torch.Generator().manual_seed(99)
    sinks = torch.randn(8, generator=g).float().to(cuda)
    got = f32(run_decode_ws(case, 0, 7, sinks))
    assert_close(got[seqs], oracle_decode(case, seqs, window_left=7, sinks=sinks)[seqs], BF16_TOL,
                 BF16_TOL, "batch 9000, window 7 + sinks")


def test_paged_decode_workspace_reuse(cuda):
    """One workspace across repeated balanced launches and interleaved fixed-partition
    launches (stale partials from an earlier call never leak into a later one)."""
    case = workloads.c3_decode(cuda, batch=9, num_heads=16, kv_heads=4, pool_blocks=256,
                               ctx_lo=0, ctx_hi=6000, seed=91)
    b, hq, d = case.q.shape
    hk = case.k_cache.shape[2]
    pb = ops.paged_decode_plan(b, hq, hk, d, case.max_seq_len, 0)
    pf = ops.paged_decode_plan(b, hq, hk, d, case.max_seq_len, 5)
    ws = torch.zeros(max(pb.workspace_bytes, pf.workspace_bytes), dtype=torch.uint8, device=cuda)
    ref = oracle_decode(case)
    for it, plan in enumerate([pb, pb, pf, pb, pf, pb]):
        out = torch.full_like(case.q, float("nan"))
        ops.paged_decode(out, case.q, case.k_cache, case.v_cache, case.block_tables,
                         case.ctx_lens, case.scale, plan.part_tokens, plan.max_parts, ws)
        torch.cuda.synchronize()
        assert_close(f32(out), ref, BF16_TOL, BF16_TOL, f"call {it} part={plan.part_tokens}")


def test_paged_decode_balanced_repeatable(cuda):
    """Repeated balanced launches on one workspace give identical bits (the schedule
    depends only on the lengths), and match the oracle."""
    case = workloads.c3_decode(cuda, batch=40, num_heads=32, kv_heads=8, pool_blocks=1024,
                               ctx_lo=1, ctx_hi=6000, seed=93)
    b, hq, d = case.q.shape
    plan = ops.paged_decode_plan(b, hq, 8, d, case.max_seq_len, 0)
    ws = torch.zeros(plan.workspace_bytes, dtype=torch.uint8, device=cuda)
    outs = []
    for _ in range(4):
        out = torch.full_like(case.q, float("nan"))
        ops.paged_decode(out, case.q, case.k_cache, case.v_cache, case.block_tables,
                         case.ctx_lens, case.scale, plan.part_tokens, plan.max_parts, ws)
        torch.cuda.synchronize()
        outs.append(out)
    for o in outs[1:]:
        assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16))
    seqs = list(range(0, b, 5))
    assert_close(f32(outs[0])[seqs], oracle_decode(case, seqs)[seqs], BF16_TOL, BF16_TOL, "C3-like")


def test_paged_decode_padded_rows_and_masked_pages(cuda):
    """ctx 0 rows (engine padding, engine.py:5405-5407) give zeros; a -1 page inside
    the context is masked instead of read."""
    ctx = [0, 300, 0, 70]
    case = workloads.c3_decode(cuda, num_heads=8, kv_heads=2, block_size=64, pool_blocks=32,
                               ctx_lens=ctx, seed=41)
    out = f32(run_decode(case))
    ref = oracle_decode(case)
    assert np.array_equal(out[0], np.zeros_like(out[0])) and np.array_equal(out[2], 0 * out[2])
    assert_close(out, ref, BF16_TOL, BF16_TOL)
    # Mask page 1 of sequence 1: tokens 64..127 drop out of its softmax.
    bt = case.block_tables.clone()
    bt[1, 1] = -1
    case.block_tables = bt
    out2 = f32(run_decode(case))
    q = f32(case.q)[1]
    keep = np.r_[0:64, 128:300]
    ids = case.block_tables[1, :5].cpu().numpy()
    ids[1] = 0
    kp = f32(case.k_cache[torch.from_numpy(ids.astype(np.int64)).to(cuda)]).reshape(-1, 2, 128)
    vp = f32(case.v_cache[torch.from_numpy(ids.astype(np.int64)).to(cuda)]).reshape(-1, 2, 128)
    ref1 = oracle.attend_one(q, kp[keep], vp[keep], case.scale)
    assert_close(out2[1], ref1, BF16_TOL, BF16_TOL, "masked page")


def test_paged_decode_fp8_small(cuda):
    _flush("paged_decode fp8 small")
    case = workloads.c5_fp8_decode(cuda, batch=3, ctx_lens=[5000, 8192, 333], seed=51)
    ref = oracle_decode(case)
    for splits in (0, 16):
        assert_close(f32(run_decode(case, splits)), ref, FP8_TOL, FP8_TOL, f"fp8 splits={splits}")


def test_paged_decode_fp8_dequant_rounding(cuda):
    """One key per sequence: the output row is that key's V row, so each element must be
    float(v8) * v_scale rounded to nearest even in bf16, bit for bit (_cast_kv_tile's
    (data.to(float32) * scale).to(q.dtype), triton_unified_attention.py:64-67)."""
    _flush("paged_decode fp8 dequant rounding")
    case = workloads.c5_fp8_decode(cuda, batch=6, ctx_lens=[1] * 6, block_size=16, seed=57)
    got = run_decode(case, 0)
    vs = case.v_scale.float().cpu()
    b, hq, d = case.q.shape
    hk = case.v_cache.shape[2]
    bt = case.block_tables.cpu()
    v8 = case.v_cache.cpu()
    for i in range(b):
        row = v8[int(bt[i, 0]), 0]  # [Hk, D], token 0 of the sequence's first page
        want = (row.float() * vs[:, None]).to(torch.bfloat16)  # RNE
        want = want.repeat_interleave(hq // hk, dim=0)
        assert torch.equal(got[i].cpu(), want), f"sequence {i}"


@pytest.fixture(scope="module")
def c5_outputs(cuda):
    """The full C5 launch (8 x 131072, fp8 KV with per-kv-head scales) under the balanced
    schedule and 16 / 32 / 64 fixed partitions."""
    _flush("paged_decode C5 fp8: GPU launches")
    case = workloads.c5_fp8_decode(cuda)
    outs = {splits: f32(run_decode(case, splits)) for splits in (0, 16, 32, 64)}
    return case, outs


@pytest.mark.parametrize("seqs", [(0, 1), (2, 3), (4, 5), (6, 7)])
def test_paged_decode_fp8_c5(c5_outputs, seqs):
    """Every C5 sequence against the oracle (two per test, so each oracle leg stays well
    inside the per-test timeout), for every schedule.  Kernel and oracle both round
    float(x) * scale to bf16 before the products (_cast_kv_tile)."""
    case, outs = c5_outputs
    _flush(f"paged_decode C5 fp8: oracle for sequences {seqs}")
    seqs = list(seqs)
    ref = oracle_decode(case, seqs=seqs)
    for splits, got in outs.items():
        assert np.isfinite(got).all()
        assert_close(got[seqs], ref[seqs], FP8_TOL, FP8_TOL, f"C5 seqs {seqs} splits={splits}")


def run_decode_ws(case, num_splits=0, window_left=-1, sinks=None):
    b, hq, d = case.q.shape
    hk = case.k_cache.shape[2]
    part, nparts, wsb = ops.paged_decode_plan(b, hq, hk, d, case.max_seq_len, num_splits)
    ws = torch.zeros(max(1, wsb), dtype=torch.uint8, device=case.q.device)
    out = torch.full_like(case.q, float("nan"))
    ops.paged_decode(out, case.q, case.k_cache, case.v_cache, case.block_tables, case.ctx_lens,
                     case.scale, part, nparts, ws, case.k_scale, case.v_scale, window_left, sinks)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("num_splits", [0, 3, 16])
@pytest.mark.parametrize("window_left", [0, 1, 15, 16, 100, 1000, 5000])
def test_paged_decode_sliding_window_and_sinks(cuda, num_splits, window_left):
    """Sliding window (flash-attn window_size = (window_left, 0)) at edges of tiles
    (16 tokens), pages (64) and partitions, with and without attention sinks, on the
    balanced schedule and on fixed partitions (some wholly before the window)."""
    _flush(f"decode window={window_left} splits={num_splits}")
    ctx = [1, 15, 16, 17, 255, 256, 257, 1000, 4000, 0, 2047]
    pool = sum((n + 63) // 64 for n in ctx) + 3
    case = workloads.c3_decode(cuda, num_heads=32, kv_heads=8, block_size=64, pool_blocks=pool,
                               ctx_lens=ctx, seed=61 + window_left)
    g = torch.Generator().manual_seed(62)
    sinks = (2 * torch.randn(32, generator=g)).float().to(cuda)
    for sk in (None, sinks):
        got = f32(run_decode_ws(case, num_splits, window_left, sk))
        ref = oracle_decode(case, window_left=window_left, sinks=sk)
        assert_close(got, ref, BF16_TOL, BF16_TOL, f"window={window_left} sinks={sk is not None}")
        assert not got[9].any()  # empty context: zero row, sinks or not


@pytest.mark.parametrize("lens,num_splits,hd", [
    ([20_000], 0, 128),          # one sequence over every range: one merge row per work-group
    ([5_000, 30_000], 0, 128),   # two, cut into ~130 and ~230 pieces
    ([3, 9_000, 0], 0, 64),      # three, with a short and an empty one
    ([8_192, 100], 128, 128),    # 128 fixed partitions
    ([12_000], 0, 256),
])
def test_paged_decode_merge_many_pieces(cuda, lens, num_splits, hd):
    """Rows cut into more pieces than one wave folds in a round: several waves per
    row fold strided subsets and are combined through LDS (with a work-group per
    row for small batches), with and without sinks, against the oracle."""
    _flush(f"decode many pieces lens={lens} splits={num_splits} D={hd}")
    bs = 256
    pool = sum((n + bs - 1) // bs for n in lens) + 2
    case = workloads.c3_decode(cuda, num_heads=16, kv_heads=4, head_dim=hd, block_size=bs,
                               pool_blocks=pool, ctx_lens=lens, seed=91 + hd)
    g = torch.Generator().manual_seed(92)
    sinks = (2 * torch.randn(16, generator=g)).float().to(cuda)
    for sk in (None, sinks):
        got = f32(run_decode_ws(case, num_splits, -1, sk))
        ref = oracle_decode(case, sinks=sk)
        assert_close(got, ref, BF16_TOL, BF16_TOL, f"lens={lens} splits={num_splits} D={hd}")
        for i, n in enumerate(lens):
            if n == 0:
                assert not got[i].any()


def test_paged_decode_sinks_c3_and_fp8(cuda):
    """Sinks at C3 size (balanced; sequences cut across work-groups merge the sink
    once) and on fp8 pages with a window, against the oracle."""
    _flush("decode sinks C3 + fp8 window")
    case = workloads.c3_decode(cuda)
    g = torch.Generator().manual_seed(63)
    sinks = (3 * torch.randn(32, generator=g)).float().to(cuda)
    got = f32(run_decode_ws(case, 0, -1, sinks))
    ctx = case.ctx_lens.cpu().numpy()
    seqs = [int(i) for i in np.argsort(ctx)[::9]]
    assert_close(got[seqs], oracle_decode(case, seqs, sinks=sinks)[seqs], BF16_TOL, BF16_TOL, "C3")
    c5 = workloads.c5_fp8_decode(cuda, batch=3, ctx_lens=[5000, 8192, 333], seed=64)
    s64 = (2 * torch.randn(64, generator=g)).float().to(cuda)
    for splits in (0, 16):
        assert_close(f32(run_decode_ws(c5, splits, 700, s64)),
                     oracle_decode(c5, window_left=700, sinks=s64), FP8_TOL, FP8_TOL,
                     f"fp8 window splits={splits}")


def test_candidate_decode_window_and_sinks_kwargs(cuda):
    """FlashAttnDecode as Attention drives it: the window from the _window_size
    attribute (attention_impl.py:242-244, :282) or the window_size kwarg, sinks as
    s_aux in the model dtype (attention_impl.py:401-406), both through forward and
    forward_store, against the oracle."""
    from fastkernels_amd.candidate.L1.flash_attn_decode import FlashAttnDecode

    ctx = [300, 77, 1024, 5]
    case = workloads.c3_decode(cuda, num_heads=16, kv_heads=4, block_size=64, pool_blocks=64,
                               ctx_lens=ctx, seed=65)
    g = torch.Generator().manual_seed(66)
    s_aux = (2 * torch.randn(16, generator=g)).to(torch.bfloat16).to(cuda)
    ref = oracle_decode(case, window_left=127, sinks=s_aux.float())
    mod = FlashAttnDecode(16, 4, 128, page_size=64)
    mod._window_size = (127, 0)
    kw = dict(block_table=case.block_tables, softmax_scale=case.scale, causal=True,
              max_seq_len=case.max_seq_len, s_aux=s_aux)
    assert_close(f32(mod(case.q, case.k_cache, case.v_cache, case.ctx_lens, **kw)), ref,
                 BF16_TOL, BF16_TOL, "attribute window")
    mod2 = FlashAttnDecode(16, 4, 128, page_size=64)
    assert_close(f32(mod2(case.q, case.k_cache, case.v_cache, case.ctx_lens,
                          window_size=(127, 0), **kw)), ref, BF16_TOL, BF16_TOL, "kwarg window")
    assert_close(f32(mod2(case.q, case.k_cache, case.v_cache, case.ctx_lens,
                          window_size=(127, 0), num_splits=4, **kw)), ref, BF16_TOL, BF16_TOL,
                 "kwarg window, 4 splits")
    # forward_store: the new rows stored at each sequence's last slot, then decode
    rows = workloads.decode_step_rows(case)
    kc, vc = case.k_cache.clone(), case.v_cache.clone()
    got = mod.forward_store(case.q, rows.key, rows.value, kc, vc, rows.slot_mapping,
                            case.ctx_lens, **kw)
    ops.store_kvcache(rows.key, rows.value, case.k_cache, case.v_cache, rows.slot_mapping)
    torch.cuda.synchronize()
    assert torch.equal(kc, case.k_cache) and torch.equal(vc, case.v_cache)
    assert_close(f32(got), oracle_decode(case, window_left=127, sinks=s_aux.float()), BF16_TOL,
                 BF16_TOL, "forward_store window + sinks")


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize("num_splits", [0, 5])
def test_candidate_decode_reference_harness_inputs(cuda, kv_dtype, num_splits):
    """FlashAttnDecode on inputs built as the reference bench builds a paged decode's:
    random caches, then ``_fix_paged_decode`` (page ids drawn with repetition, so
    sequences share pages and a page may recur within one; lengths up to the
    table's reach).  Judged by the reference's acceptance rule against the oracle
    rounded to the output dtype (PASSED), and by this suite's per-element bar."""
    from fastkernels_amd.candidate.L1.flash_attn_decode import FlashAttnDecode

    _flush(f"candidate decode, harness inputs {kv_dtype} splits={num_splits}")
    fp8 = kv_dtype == torch.float8_e4m3fn
    g = torch.Generator().manual_seed(43 + num_splits)
    b, hq, hk, d, nb, bs, width = 12, 32, 8, 128, 20, 64, 14
    q = torch.randn(b, hq, d, generator=g).to(torch.bfloat16).to(cuda)
    k = torch.randn(nb, bs, hk, d, generator=g).to(cuda)
    v = torch.randn(nb, bs, hk, d, generator=g).to(cuda)
    scales = {}
    if fp8:
        ks = (0.01 + 0.09 * torch.rand(hk, generator=g)).to(cuda)
        vs = (0.01 + 0.09 * torch.rand(hk, generator=g)).to(cuda)
        k, v = workloads.quantize_fp8(k, ks), workloads.quantize_fp8(v, vs)  # as C5
        scales = {"k_scale": ks, "v_scale": vs}
    else:
        k, v = k.to(torch.bfloat16), v.to(torch.bfloat16)
    kw = {"k_cache": k, "v_cache": v, "block_table": torch.zeros(b, width, dtype=torch.int32),
          "cache_seqlens": torch.zeros(b, dtype=torch.int32), "max_seq_len": 0}
    fix_paged_decode(kw, generator=g, page_dim=1)
    bt = kw["block_table"].cpu().numpy()
    assert any(len(set(row.tolist())) < width for row in bt)  # pages recur within a sequence
    mod = FlashAttnDecode(hq, hk, d, page_size=bs)
    out = mod(q, k, v, kw["cache_seqlens"], block_table=kw["block_table"],
              max_seq_len=kw["max_seq_len"], softmax_scale=d ** -0.5, causal=True,
              num_splits=num_splits, **scales)
    torch.cuda.synchronize()
    raw = (lambda t: t.view(torch.uint8).cpu().numpy()) if fp8 else f32
    ref = oracle.paged_decode(f32(q), raw(k), raw(v), bt, kw["cache_seqlens"].cpu().numpy(),
                              d ** -0.5, *(s.cpu().numpy() for s in scales.values()))
    got = f32(out)
    status, max_abs, _, matched, detail = oracle.compare(got, oracle.round_to(ref, "bf16"), "bf16")
    assert status == oracle.PASSED, (status, max_abs, matched, detail)
    tol = FP8_TOL if fp8 else BF16_TOL
    assert_close(got, ref, tol, tol, "harness inputs")


# ---------------------------------------------------------------------------
# Candidate classes (drop-in surface) and the C4 chain
# ---------------------------------------------------------------------------
@pytest.fixture(scope="module")
def c4_chain_run(cuda):
    """C4: add+RMSNorm -> rotary -> store_kvcache -> paged decode -> SiLU-and-mul through
    the candidate classes on the full C4 inputs.  Returns the inputs, each op's input
    snapshot and each op's output; the tests below check every output against the
    oracle."""
    _flush("chain C4: GPU launches")
    from fastkernels_amd.candidate.L1.flash_attn_decode import FlashAttnDecode
    from fastkernels_amd.candidate.L1.rms_norm import RMSNorm
    from fastkernels_amd.candidate.L1.rotary_emb import RotaryEmbedding
    from fastkernels_amd.candidate.L1.silu_and_mul import SiluAndMul
    from fastkernels_amd.candidate.L1.store_kvcache import StoreKVCache

    c = workloads.c4_chain(cuda)
    t, hq, hk, d = 256, 32, 8, 128
    res = {"c": c}
    norm = RMSNorm(4096).to(cuda)
    norm.weight.data.copy_(c.norm_weight.float())
    res["norm_out"] = norm(c.hidden.clone(), c.residual.clone())

    rope = RotaryEmbedding(d, c.max_position, c.rope_theta).to(cuda)
    res["cos_sin"] = f32(rope.cos_sin_cache)
    qkv = c.qkv.clone()
    q, k, v = qkv[:, :hq * d], qkv[:, hq * d:(hq + hk) * d], qkv[:, (hq + hk) * d:]
    res["q_in"], res["k_in"] = f32(q), f32(k)
    rope(c.positions, q, k)
    res["q"], res["k"] = q, k

    dec = c.decode
    StoreKVCache()(k.view(t, hk, d), v.view(t, hk, d), dec.k_cache, dec.v_cache, c.slot_mapping)
    attn = FlashAttnDecode(hq, hk, d, page_size=256)
    o = attn(q.view(t, hq, d), dec.k_cache, dec.v_cache, cache_seqlens=dec.ctx_lens,
             block_table=dec.block_tables, softmax_scale=dec.scale, causal=True,
             max_seq_len=dec.max_seq_len)
    dec.q = q.view(t, hq, d)
    res["attn"] = f32(o)
    res["act"] = SiluAndMul()(c.gate_up)
    torch.cuda.synchronize()
    return res


def test_candidates_chain_c4(c4_chain_run):
    """The C4 chain's norm, rotary, store and SiLU outputs against the oracle (the
    residual and the stored cache rows bit-exact)."""
    _flush("chain C4: norm / rotary / store / silu")
    res = c4_chain_run
    c = res["c"]
    t, hk, d = 256, 8, 128
    hn, rn = res["norm_out"]
    ref_h, ref_r = oracle.rms_norm(f32(c.hidden), f32(c.norm_weight), 1e-6, "bf16",
                                   residual=f32(c.residual))
    assert np.array_equal(f32(rn), ref_r)
    assert_close(f32(hn), ref_h, BF16_TOL, BF16_TOL, "norm")

    ref_q, ref_k = oracle.rotary(c.positions.cpu().numpy(), res["q_in"], res["k_in"], d,
                                 res["cos_sin"], True, "bf16")
    assert_close(f32(res["q"]), ref_q, BF16_TOL, BF16_TOL, "rope q")
    assert_close(f32(res["k"]), ref_k, BF16_TOL, BF16_TOL, "rope k")

    dec = c.decode
    rows = c.slot_mapping
    kflat = dec.k_cache.view(-1, hk * d)
    assert torch.equal(kflat[rows].view(torch.int16), res["k"].contiguous().view(torch.int16))
    vflat = dec.v_cache.view(-1, hk * d)
    v = c.qkv[:, (32 + hk) * d:]
    assert torch.equal(vflat[rows].view(torch.int16), v.contiguous().view(torch.int16))

    assert_close(f32(res["act"]), oracle.silu_and_mul(f32(c.gate_up), "bf16"), BF16_TOL,
                 BF16_TOL, "silu")


@pytest.mark.parametrize("first", [0, 64, 128, 192])
def test_candidates_chain_c4_decode(c4_chain_run, first):
    """The C4 chain's paged decode (B = 256, ctx U[256, 4096], over the caches the
    chain's store wrote): every sequence against the oracle, 64 per test."""
    res = c4_chain_run
    seqs = list(range(first, first + 64))
    _flush(f"chain C4: decode oracle for sequences {first}..{first + 63}")
    ref = oracle_decode(res["c"].decode, seqs)
    got = res["attn"]
    assert np.isfinite(got[seqs]).all()
    assert_close(got[seqs], ref[seqs], BF16_TOL, BF16_TOL, f"C4 decode seqs {first}..")


def test_flash_attn_decode_defaults_no_sync(cuda):
    """max_seq_len omitted: bound from the block table width, no host sync needed."""
    from fastkernels_amd.candidate.L1.flash_attn_decode import FlashAttnDecode

    case = workloads.c3_decode(cuda, batch=5, num_heads=16, kv_heads=4, pool_blocks=64,
                               ctx_lo=10, ctx_hi=3000, seed=61)
    attn = FlashAttnDecode(16, 4, 128)
    o = attn(case.q, case.k_cache, case.v_cache, cache_seqlens=case.ctx_lens,
             block_table=case.block_tables)
    assert_close(f32(o), oracle_decode(case), BF16_TOL, BF16_TOL)
    assert math.isclose(case.scale, 1 / math.sqrt(128))


# ---------------------------------------------------------------------------
# merge_attn_states
# ---------------------------------------------------------------------------
def _merge_inputs(t, h, d, dtype, cuda, seed, specials=True):
    g = torch.Generator().manual_seed(seed)
    po = torch.randn(t, h, d, generator=g).to(dtype)
    so = torch.randn(t, h, d, generator=g).to(dtype)
    pl = (3 * torch.randn(h, t, generator=g)).float()
    sl = (3 * torch.randn(h, t, generator=g)).float()
    if specials and t >= 4:
        pl[0, 0] = -math.inf                    # empty prefix
        sl[0, 1] = -math.inf                    # empty suffix
        pl[h - 1, 2] = sl[h - 1, 2] = -math.inf  # both empty: the prefix rows are copied
        pl[h - 1, 3] = math.inf                 # +inf read as -inf
        sl[0, 3] = 40.0                         # far apart: one weight underflows
    return po.to(cuda), pl.to(cuda), so.to(cuda), sl.to(cuda)


def _check_merge(out, out_lse, po, pl, so, sl, dtype, prefill=None):
    ref, ref_lse = oracle.merge_attn_states(f32(po), f32(pl), f32(so), f32(sl), _DT[dtype], prefill)
    tol = (BF16_TOL, BF16_TOL) if dtype != torch.float32 else (1e-5, 1e-3)
    assert_close(f32(out), ref, *tol, what="merge out")
    # copied rows are bit copies of the input rows
    both = torch.isinf(pl) & torch.isinf(sl)
    n = po.shape[0] if prefill is None else prefill
    for hh, tt in both.nonzero().tolist():
        if tt < n:
            assert torch.equal(out[tt, hh], po[tt, hh])
    if n < po.shape[0]:
        assert torch.equal(out[n:], so[n:])
    if out_lse is not None:
        got = f32(out_lse)
        assert np.array_equal(np.isneginf(got), np.isneginf(ref_lse))
        fin = np.isfinite(ref_lse)
        assert_close(got[fin], ref_lse[fin], 1e-5, 1e-5, what="merge lse")
        if n < po.shape[0]:
            assert torch.equal(out_lse[:, n:], sl[:, n:])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("t,h,d", [(64, 32, 128), (5, 3, 100), (33, 8, 256), (1, 1, 8)])
@pytest.mark.parametrize("with_lse", [True, False])
def test_merge_attn_states(cuda, dtype, t, h, d, with_lse):
    _flush(f"merge {dtype} t={t} h={h} d={d} lse={with_lse}")
    po, pl, so, sl = _merge_inputs(t, h, d, dtype, cuda, seed=t * 7 + d)
    out = torch.full_like(po, float("nan"))
    out_lse = torch.full((h, t), float("nan"), device=cuda) if with_lse else None
    ops.merge_attn_states(out, po, pl, so, sl, out_lse)
    torch.cuda.synchronize()
    _check_merge(out, out_lse, po, pl, so, sl, dtype)


def test_merge_attn_states_prefill_tokens_and_strides(cuda):
    """Suffix-only tail tokens, and strided [T, H, D] views (a slice of a wider
    buffer for the inputs, a head-padded output)."""
    t, h, d = 48, 16, 128
    dtype = torch.bfloat16
    _flush("merge strided + prefill_tokens_with_context=30")
    g = torch.Generator().manual_seed(5)
    wide = torch.randn(2, t, h, d + 64, generator=g).to(dtype).to(cuda)
    po, so = wide[0, :, :, :d], wide[1, :, :, :d]
    _, pl, _, sl = _merge_inputs(t, h, d, dtype, cuda, seed=6)
    out_buf = torch.full((t, h, d + 32), float("nan"), dtype=dtype, device=cuda)
    out = out_buf[:, :, :d]
    out_lse = torch.full((h, t), float("nan"), device=cuda)
    ops.merge_attn_states(out, po, pl, so, sl, out_lse, prefill_tokens_with_context=30)
    torch.cuda.synchronize()
    _check_merge(out, out_lse, po, pl, so, sl, dtype, prefill=30)
    assert torch.isnan(out_buf[:, :, d:].float()).all(), "padding written"


def test_merge_attn_states_two_halves_equal_whole(cuda):
    """Attention over 2000 keys split at 700 and merged on the GPU equals attention
    over all of them (torch fp32 on the device computes the halves and the whole)."""
    t, h, d, n, cut = 32, 8, 128, 2000, 700
    _flush("merge halves == whole")
    g = torch.Generator().manual_seed(8)
    q = torch.randn(t, h, 1, d, generator=g).to(cuda)
    k = torch.randn(t, h, n, d, generator=g).to(cuda)
    v = torch.randn(t, h, n, d, generator=g).to(cuda)
    sc = d ** -0.5
    s = (q @ k.transpose(-1, -2).contiguous())[:, :, 0] * sc  # [t, h, n]

    def attend(lo, hi):
        p = torch.softmax(s[..., lo:hi], dim=-1)
        o = (p.unsqueeze(-2) @ v[:, :, lo:hi])[:, :, 0]
        return o.bfloat16().contiguous(), torch.logsumexp(s[..., lo:hi], -1).T.contiguous()

    (po, pl), (so, sl), (whole, whole_lse) = attend(0, cut), attend(cut, n), attend(0, n)
    out = torch.empty_like(po)
    out_lse = torch.empty_like(pl)
    ops.merge_attn_states(out, po, pl, so, sl, out_lse)
    torch.cuda.synchronize()
    assert_close(f32(out), f32(whole), BF16_TOL, BF16_TOL, what="halves vs whole")
    assert_close(f32(out_lse), f32(whole_lse), 1e-4, 1e-5, what="lse halves vs whole")


def test_merge_attn_states_candidate(cuda):
    from fastkernels_amd.candidate.L1.merge_attn_states import MergeAttnStates
    t, h, d = 16, 8, 128
    po, pl, so, sl = _merge_inputs(t, h, d, torch.bfloat16, cuda, seed=9)
    out = torch.empty_like(po)
    out_lse = torch.empty_like(pl)
    MergeAttnStates()(out, po, pl, so, sl, out_lse)
    torch.cuda.synchronize()
    _check_merge(out, out_lse, po, pl, so, sl, torch.bfloat16)


@pytest.mark.parametrize("dtype,t,h,d,prefill", [
    (torch.bfloat16, 300, 16, 128, None),  # vector path, 16 lanes a head
    (torch.bfloat16, 64, 8, 512, 40),      # 64 lanes a head; a suffix-only tail
    (torch.float16, 33, 4, 72, None),      # 9 vectors a head
    (torch.float32, 50, 4, 128, 20),
    (torch.bfloat16, 20, 3, 100, None),    # head 100: the scalar path
])
def test_merge_attn_states_fp8_output(cuda, dtype, t, h, d, prefill):
    """fp8 e4m3fn output (output_scale; merge_attn_states.cu's USE_FP8_OUTPUT form): the
    copied rows (both sides empty, tokens past prefill_tokens_with_context) equal the
    oracle's codes bit for bit; every merged value is the oracle's code or a neighbour
    (the fp32 merge rounds once more in fp8), 99% of them exactly; the lse is as with
    a bf16 output.  Values beyond +-448 saturate."""
    _flush(f"merge_attn_states fp8 output {dtype} {t}x{h}x{d} prefill={prefill}")
    po, pl, so, sl = _merge_inputs(t, h, d, dtype, cuda, seed=31 + d)
    po, so = po * 100, so * 100  # some values past 448 * scale
    scale = torch.tensor([0.5], dtype=torch.float32, device=cuda)
    out = torch.empty(t, h, d, dtype=torch.float8_e4m3fn, device=cuda)
    out_lse = torch.empty_like(pl)
    ops.merge_attn_states(out, po, pl, so, sl, out_lse, prefill, scale)
    torch.cuda.synchronize()
    codes, ref_lse = oracle.merge_attn_states(f32(po), f32(pl), f32(so), f32(sl), _DT[dtype],
                                              prefill, output_scale=0.5)
    got = out.view(torch.uint8).cpu().numpy()
    both = (torch.isinf(pl) & torch.isinf(sl)).cpu().numpy().T  # [t, h]
    n = t if prefill is None else prefill
    copied = np.zeros((t, h), bool)
    copied[:n] = both[:n]
    copied[n:] = True
    assert np.array_equal(got[copied], codes[copied]), "copied rows"
    dg, dr = oracle.fp8_e4m3fn_decode(got[~copied]), oracle.fp8_e4m3fn_decode(codes[~copied])
    step = np.maximum(np.abs(dr) * 2.0 ** -3, 2.0 ** -9)
    assert (np.abs(dg - dr) <= step).all(), "merged values more than one e4m3fn step apart"
    assert (got[~copied] == codes[~copied]).mean() > 0.99
    assert (np.abs(oracle.fp8_e4m3fn_decode(got)) == 448.0).any()  # saturation exercised
    fin = np.isfinite(ref_lse)
    assert np.array_equal(np.isneginf(f32(out_lse)), np.isneginf(ref_lse))
    assert_close(f32(out_lse)[fin], ref_lse[fin], 1e-5, 1e-5, what="merge lse")


def test_merge_attn_states_candidate_fp8_output(cuda):
    """The candidate function with output_scale (the reference's keyword) into an fp8
    output; a missing scale is refused."""
    from fastkernels_amd.candidate.L1.merge_attn_states import merge_attn_states
    t, h, d = 16, 8, 128
    po, pl, so, sl = _merge_inputs(t, h, d, torch.bfloat16, cuda, seed=19)
    out = torch.empty(t, h, d, dtype=torch.float8_e4m3fn, device=cuda)
    merge_attn_states(out, po, pl, so, sl, output_scale=torch.tensor([0.125], device=cuda))
    torch.cuda.synchronize()
    codes, _ = oracle.merge_attn_states(f32(po), f32(pl), f32(so), f32(sl), "bf16",
                                        output_scale=0.125)
    dg = oracle.fp8_e4m3fn_decode(out.view(torch.uint8).cpu().numpy())
    dr = oracle.fp8_e4m3fn_decode(codes)
    assert (np.abs(dg - dr) <= np.maximum(np.abs(dr) * 2.0 ** -3, 2.0 ** -9)).all()
    with pytest.raises(ValueError, match="output_scale"):
        merge_attn_states(out, po, pl, so, sl)


# ---------------------------------------------------------------------------
# store_kvcache with a dtype conversion (bf16/fp16/fp32 key -> fp8 / bf16 cache)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("src", [torch.bfloat16, torch.float16, torch.float32])
def test_store_kvcache_convert_to_fp8(cuda, src):
    """The conversion tl.store applies (round to nearest even, saturating at +-448,
    NaN kept) against the oracle's encoder, bit-exact, with ties, subnormals,
    saturation, infinities and NaN planted."""
    _flush(f"store_kvcache convert {src} -> fp8")
    g = torch.Generator().manual_seed(90)
    n, hk, d = 300, 8, 128
    key = (torch.randn(n, hk, d, generator=g) * 40).to(src)
    val = (torch.randn(n, hk, d, generator=g) * 1e-3).to(src)  # subnormal range of e4m3fn
    special = torch.tensor([0.0, -0.0, 447.0, 448.0, 460.0, 464.0, 1e4, float("inf"), float("-inf"),
                            float("nan"), 2.0 ** -9, 1.5 * 2.0 ** -9, 2.0 ** -10, 0.0068359375,
                            1.0625, 1.1875, -3.25 * 2.0 ** -8, 240.0, 232.0])
    key.view(-1)[:special.numel()] = special.to(src)
    slots = torch.randperm(64 * 16, generator=g)[:n].to(torch.int64)
    slots[7] = -1
    kc = torch.zeros(64, 16, hk, d, dtype=torch.float8_e4m3fn)
    vc = torch.zeros_like(kc)
    key_d, val_d, kc_d, vc_d, sl_d = (t.to(cuda) for t in (key, val, kc, vc, slots))
    ops.store_kvcache(key_d, val_d, kc_d, vc_d, sl_d)
    torch.cuda.synchronize()
    ek = oracle.fp8_e4m3fn_encode(key.float().numpy())
    ev = oracle.fp8_e4m3fn_encode(val.float().numpy())
    zk = np.zeros((64 * 16, hk * d), np.uint8)
    zv = np.zeros_like(zk)
    ok = slots.numpy() >= 0
    zk[slots.numpy()[ok]] = ek.reshape(n, -1)[ok]
    zv[slots.numpy()[ok]] = ev.reshape(n, -1)[ok]
    assert np.array_equal(kc_d.view(torch.uint8).cpu().numpy().reshape(-1, hk * d), zk)
    assert np.array_equal(vc_d.view(torch.uint8).cpu().numpy().reshape(-1, hk * d), zv)


def test_store_kvcache_convert_f32_to_bf16(cuda):
    g = torch.Generator().manual_seed(91)
    key = torch.randn(33, 2, 64, generator=g).to(cuda)
    val = torch.randn(33, 2, 64, generator=g).to(cuda)
    kc = torch.zeros(8, 16, 2, 64, dtype=torch.bfloat16, device=cuda)
    vc = torch.zeros_like(kc)
    slots = torch.randperm(128, generator=g)[:33].to(torch.int32).to(cuda)
    ops.store_kvcache(key, val, kc, vc, slots)
    torch.cuda.synchronize()
    kf = kc.view(-1, 128)[slots.long()]
    assert torch.equal(kf, key.view(33, -1).bfloat16())  # torch's RNE cast
    assert torch.equal(vc.view(-1, 128)[slots.long()], val.view(33, -1).bfloat16())
