"""Seeded synthetic inputs for the five decode-step configurations (C1-C5).

These are the input builders of the benchmark and the parity tests: the same
seed gives the same tensors.  Value distributions follow the benchmark
configurations of this path:

C1  fused add+RMSNorm: x, residual [256, 1024] ~ N(0,1), weight = 1 + 0.1 N(0,1), eps 1e-6.
C2  store_kvcache: K, V [4096, 8, 128] bf16 ~ N(0,1); caches [2048, 256, 8, 128] zero;
    slot_mapping int64 = 4096 distinct slots of a seeded permutation of 0..524287,
    5% (205) set to -1.
C3  paged decode, Qwen3-8B shape: q [64, 32, 128] bf16; Hk 8; block 256; ctx int32
    ~ U[512, 8192]; block tables from a seeded permutation of a 4096-block pool;
    KV bf16 ~ N(0,1); scale 1/sqrt(128).
C4  decode-layer chain, batch 256, Qwen3-8B dims: add+RMSNorm [256, 4096] -> rotary
    (theta 1e6, positions = ctx_len) on q/k -> store_kvcache -> paged decode
    (ctx ~ U[256, 4096]) -> SiLU-and-mul on [256, 2*12288].
C5  fp8-KV long context: 8 seqs x 131072; q [8, 64, 128] bf16; Hk 8; block 256;
    KV e4m3fn from N(0,1)/scale with saturation; per-kv-head fp32 scales ~ U[0.01, 0.1].

The decode metadata follows the reference engine's conventions
(ModelRunner.prepare_decode, fastkernels/infra/engine.py:5001-5076): block tables
int32 padded with -1 past each sequence's pages, context lengths int32.
Large tensors are drawn on the target device with a device generator.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

SEED = 200  # the reference harness's DEFAULT_SEED (fastkernels/bench.py:139)


def _gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _randn(shape, device, seed, dtype=torch.bfloat16) -> torch.Tensor:
    return torch.randn(shape, generator=_gen(device, seed), device=device,
                       dtype=torch.float32).to(dtype)


# ---------------------------------------------------------------------------
# C1
# ---------------------------------------------------------------------------
@dataclass
class NormCase:
    x: torch.Tensor
    residual: torch.Tensor
    weight: torch.Tensor
    eps: float = 1e-6


def c1_norm(device="cpu", dtype=torch.bfloat16, tokens=256, hidden=1024, seed=SEED) -> NormCase:
    g = _gen("cpu", seed)
    x = torch.randn(tokens, hidden, generator=g)
    r = torch.randn(tokens, hidden, generator=g)
    w = 1.0 + 0.1 * torch.randn(hidden, generator=g)
    return NormCase(x.to(device, dtype), r.to(device, dtype), w.to(device, dtype))


# ---------------------------------------------------------------------------
# C2
# ---------------------------------------------------------------------------
@dataclass
class StoreCase:
    key: torch.Tensor
    value: torch.Tensor
    k_cache: torch.Tensor
    v_cache: torch.Tensor
    slot_mapping: torch.Tensor


def c2_store(device="cpu", tokens=4096, num_blocks=2048, block_size=256, kv_heads=8,
             head_dim=128, skip_frac=0.05, seed=SEED, slot_dtype=torch.int64) -> StoreCase:
    g = _gen("cpu", seed)
    key = torch.randn(tokens, kv_heads, head_dim, generator=g).to(torch.bfloat16)
    value = torch.randn(tokens, kv_heads, head_dim, generator=g).to(torch.bfloat16)
    n_slots = num_blocks * block_size
    slots = torch.randperm(n_slots, generator=g)[:tokens].to(torch.int64)
    n_skip = int(round(skip_frac * tokens))
    skip = torch.randperm(tokens, generator=g)[:n_skip]
    slots[skip] = -1
    shape = (num_blocks, block_size, kv_heads, head_dim)
    return StoreCase(key.to(device), value.to(device),
                     torch.zeros(shape, dtype=torch.bfloat16, device=device),
                     torch.zeros(shape, dtype=torch.bfloat16, device=device),
                     slots.to(slot_dtype).to(device))


# ---------------------------------------------------------------------------
# C3 / C5 (paged decode)
# ---------------------------------------------------------------------------
@dataclass
class DecodeCase:
    q: torch.Tensor             # [B, Hq, D] bf16
    k_cache: torch.Tensor       # [num_blocks, block_size, Hk, D] bf16 or float8_e4m3fn
    v_cache: torch.Tensor
    block_tables: torch.Tensor  # [B, max_blocks] int32, -1 padded
    ctx_lens: torch.Tensor      # [B] int32
    scale: float
    k_scale: torch.Tensor | None = None  # [Hk] float32 (fp8 only)
    v_scale: torch.Tensor | None = None

    @property
    def max_seq_len(self) -> int:
        return int(self.ctx_lens.max().item()) if self.ctx_lens.numel() else 0

    def algorithmic_bytes(self) -> int:
        """K+V bytes actually attended + q + out + block-table entries used + ctx."""
        b, hq, d = self.q.shape
        hk = self.k_cache.shape[2]
        bs = self.k_cache.shape[1]
        kv_elt = self.k_cache.element_size()
        ctx = self.ctx_lens.to(torch.int64)
        total = int(ctx.sum().item())
        pages = int(((ctx + bs - 1) // bs).sum().item())
        return (2 * total * hk * d * kv_elt + 2 * b * hq * d * self.q.element_size()
                + 4 * pages + 4 * b)


def make_block_tables(ctx_lens: torch.Tensor, block_size: int, pool_blocks: int,
                      g: torch.Generator) -> torch.Tensor:
    """Non-overlapping page ids per sequence from a seeded permutation of the pool,
    padded with -1 (engine.py:1974-1975)."""
    pages = [(int(n) + block_size - 1) // block_size for n in ctx_lens.tolist()]
    need = sum(pages)
    if need > pool_blocks:
        raise ValueError(f"pool of {pool_blocks} blocks cannot hold {need} pages")
    perm = torch.randperm(pool_blocks, generator=g).to(torch.int32)
    width = max(1, max(pages) if pages else 1)
    bt = torch.full((len(pages), width), -1, dtype=torch.int32)
    off = 0
    for i, p in enumerate(pages):
        bt[i, :p] = perm[off:off + p]
        off += p
    return bt


def c3_decode(device="cpu", batch=64, num_heads=32, kv_heads=8, head_dim=128, block_size=256,
              pool_blocks=4096, ctx_lo=512, ctx_hi=8192, seed=SEED,
              ctx_lens: list[int] | None = None) -> DecodeCase:
    g = _gen("cpu", seed)
    if ctx_lens is None:
        ctx = torch.randint(ctx_lo, ctx_hi + 1, (batch,), generator=g, dtype=torch.int64)
    else:
        ctx = torch.tensor(ctx_lens, dtype=torch.int64)
        batch = len(ctx_lens)
    bt = make_block_tables(ctx, block_size, pool_blocks, g)
    q = torch.randn(batch, num_heads, head_dim, generator=g).to(torch.bfloat16)
    shape = (pool_blocks, block_size, kv_heads, head_dim)
    k_cache = _randn(shape, device, seed + 1)
    v_cache = _randn(shape, device, seed + 2)
    return DecodeCase(q.to(device), k_cache, v_cache, bt.to(device),
                      ctx.to(torch.int32).to(device), 1.0 / math.sqrt(head_dim))


def quantize_fp8(x: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """x / scale[kv_head] with saturation to +-448, cast to float8_e4m3fn."""
    y = x.float() / scale.view(1, 1, -1, 1)
    return y.clamp_(-448.0, 448.0).to(torch.float8_e4m3fn)


def c5_fp8_decode(device="cpu", batch=8, num_heads=64, kv_heads=8, head_dim=128,
                  block_size=256, ctx=131072, pool_blocks=None, seed=SEED,
                  ctx_lens: list[int] | None = None) -> DecodeCase:
    g = _gen("cpu", seed)
    ctx_t = (torch.full((batch,), ctx, dtype=torch.int64) if ctx_lens is None
             else torch.tensor(ctx_lens, dtype=torch.int64))
    batch = ctx_t.numel()
    pages = int(((ctx_t + block_size - 1) // block_size).sum().item())
    pool = pool_blocks or pages
    bt = make_block_tables(ctx_t, block_size, pool, g)
    q = torch.randn(batch, num_heads, head_dim, generator=g).to(torch.bfloat16)
    k_scale = (0.01 + 0.09 * torch.rand(kv_heads, generator=g)).float()
    v_scale = (0.01 + 0.09 * torch.rand(kv_heads, generator=g)).float()
    shape = (pool, block_size, kv_heads, head_dim)
    kd, vd = k_scale.to(device), v_scale.to(device)
    k_cache = quantize_fp8(_randn(shape, device, seed + 1, torch.float32), kd)
    v_cache = quantize_fp8(_randn(shape, device, seed + 2, torch.float32), vd)
    return DecodeCase(q.to(device), k_cache, v_cache, bt.to(device),
                      ctx_t.to(torch.int32).to(device), 1.0 / math.sqrt(head_dim), kd, vd)


@dataclass
class StepRows:
    """The new token of each sequence in a decode step (Attention.forward_impl input)."""
    key: torch.Tensor           # [B, Hk, D], the cache dtype
    value: torch.Tensor
    slot_mapping: torch.Tensor  # [B] int64: the slot of position ctx - 1


def decode_step_rows(case: DecodeCase, seed: int = SEED + 20) -> StepRows:
    """Random new K/V rows and the slots the engine's decode step gives them:
    slot = block_table[b][(ctx-1) // bs] * bs + (ctx-1) % bs (engine.py:5020-5024),
    -1 for sequences without context."""
    b, _, d = case.q.shape
    hk, bs = case.k_cache.shape[2], case.k_cache.shape[1]
    g = _gen("cpu", seed)
    key = torch.randn(b, hk, d, generator=g)
    value = torch.randn(b, hk, d, generator=g)
    dev = case.q.device
    if case.k_cache.dtype == torch.float8_e4m3fn:
        key = quantize_fp8(key.to(dev).view(b, 1, hk, d), case.k_scale).view(b, hk, d)
        value = quantize_fp8(value.to(dev).view(b, 1, hk, d), case.v_scale).view(b, hk, d)
    else:
        key, value = key.to(case.k_cache.dtype).to(dev), value.to(case.v_cache.dtype).to(dev)
    ctx = case.ctx_lens.to("cpu").to(torch.int64)
    bt = case.block_tables.to("cpu").to(torch.int64)
    last = (ctx - 1).clamp(min=0)
    slots = bt[torch.arange(b), last // bs] * bs + last % bs
    slots = torch.where(ctx > 0, slots, torch.full_like(slots, -1))
    return StepRows(key, value, slots.to(dev))


# ---------------------------------------------------------------------------
# C4 (chain)
# ---------------------------------------------------------------------------
@dataclass
class ChainCase:
    hidden: torch.Tensor     # [T, 4096]
    residual: torch.Tensor   # [T, 4096]
    norm_weight: torch.Tensor
    qkv: torch.Tensor        # [T, (Hq + 2 Hk) * D] (q/k/v are strided views of it)
    positions: torch.Tensor  # [T] int64 = ctx_len
    gate_up: torch.Tensor    # [T, 2 * 12288]
    decode: DecodeCase       # caches / tables; ctx includes the token being stored
    slot_mapping: torch.Tensor  # [T] int64: last slot of each sequence
    rope_theta: float = 1e6
    max_position: int = 40960


def c4_chain(device="cpu", tokens=256, hidden=4096, num_heads=32, kv_heads=8, head_dim=128,
             inter=12288, block_size=256, pool_blocks=4096, ctx_lo=256, ctx_hi=4096,
             seed=SEED) -> ChainCase:
    dec = c3_decode(device, batch=tokens, num_heads=num_heads, kv_heads=kv_heads,
                    head_dim=head_dim, block_size=block_size, pool_blocks=pool_blocks,
                    ctx_lo=ctx_lo, ctx_hi=ctx_hi, seed=seed)
    g = _gen("cpu", seed + 10)
    h = torch.randn(tokens, hidden, generator=g).to(torch.bfloat16)
    r = torch.randn(tokens, hidden, generator=g).to(torch.bfloat16)
    w = (1.0 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16)
    qkv = torch.randn(tokens, (num_heads + 2 * kv_heads) * head_dim, generator=g).to(torch.bfloat16)
    gu = torch.randn(tokens, 2 * inter, generator=g).to(torch.bfloat16)
    ctx = dec.ctx_lens.to("cpu").to(torch.int64)
    bt = dec.block_tables.to("cpu").to(torch.int64)
    last = ctx - 1
    slots = bt[torch.arange(tokens), last // block_size] * block_size + last % block_size
    return ChainCase(h.to(device), r.to(device), w.to(device), qkv.to(device),
                     ctx.to(device), gu.to(device), dec, slots.to(device))
