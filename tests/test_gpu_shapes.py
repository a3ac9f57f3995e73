"""GPU parity of paged decode at the other shapes the reference builds FlashAttnDecode
with: head sizes 64 and 256, and query groups above 16 (several 16-column waves per kv
head), through the C ABI against the CPU oracle.

- Qwen3-Next full attention: Hq 16, Hk 2, head_dim 256 (L2/qwen3_next_attention.py:148-150).
- Whisper self-attention: Hq = Hk, head_dim 64 (L2/whisper_attention.py:185-190).
- A gpt-oss-like layer: Hq 64, Hk 8, head_dim 64, a 128-token sliding window and sinks
  (the window_size / s_aux arguments of Attention._forward_pure, attention_impl.py:401-434).
- Groups of 32, 40 and 71 query heads per kv head (the reference boundary accepts any
  num_heads % num_kv_heads == 0, flash_attn_decode.py:22-42).

Bars as in test_gpu_parity: bf16 within atol = rtol = 1e-2, fp8 KV within 3e-2; the
fused store + decode launch bit-identical to the two separate calls.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from fastkernels_amd import ops, workloads
from test_gpu_parity import BF16_TOL, FP8_TOL, assert_close, f32, oracle_decode, run_decode

pytestmark = pytest.mark.gpu

SHAPES = [
    # (label, hq, hk, head_dim)
    ("qwen3-next", 16, 2, 256),
    ("whisper", 20, 20, 64),
    ("gpt-oss", 64, 8, 64),
    ("gqa32", 64, 2, 128),
    ("gqa40-d256", 40, 1, 256),
    ("mqa71-d64", 71, 1, 64),
]


def _flush(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("label,hq,hk,d", SHAPES)
@pytest.mark.parametrize("num_splits", [0, 3])
def test_decode_shapes_bf16(cuda, label, hq, hk, d, num_splits):
    _flush(f"decode shape {label} hq={hq} hk={hk} d={d} splits={num_splits}")
    case = workloads.c3_decode(cuda, batch=7, num_heads=hq, kv_heads=hk, head_dim=d,
                               block_size=64, pool_blocks=512, ctx_lo=1, ctx_hi=2500,
                               seed=hq * 1000 + hk * 10 + d)
    ref = oracle_decode(case)
    got = f32(run_decode(case, num_splits))
    assert_close(got, ref, BF16_TOL, BF16_TOL, f"{label} splits={num_splits}")


@pytest.mark.parametrize("label,hq,hk,d", [SHAPES[0], SHAPES[2], SHAPES[4]])
def test_decode_shapes_fp8(cuda, label, hq, hk, d):
    _flush(f"decode shape fp8 {label}")
    case = workloads.c5_fp8_decode(cuda, num_heads=hq, kv_heads=hk, head_dim=d,
                                   ctx_lens=[3000, 17, 700, 4096], seed=hq + d)
    ref = oracle_decode(case)
    for splits in (0, 5):
        assert_close(f32(run_decode(case, splits)), ref, FP8_TOL, FP8_TOL,
                     f"{label} fp8 splits={splits}")


def test_decode_d256_full_batch(cuda):
    """Qwen3-Next shape at a serving batch: 64 sequences of 512..8192 tokens, balanced
    schedule, every sequence against the oracle."""
    _flush("decode qwen3-next batch 64")
    case = workloads.c3_decode(cuda, batch=64, num_heads=16, kv_heads=2, head_dim=256,
                               pool_blocks=4096, seed=77)
    assert_close(f32(run_decode(case)), oracle_decode(case), BF16_TOL, BF16_TOL, "d256 b64")


@pytest.mark.parametrize("window_left", [0, 127, 1000])
def test_decode_d64_window_and_sinks(cuda, window_left):
    _flush(f"decode gpt-oss window={window_left}")
    case = workloads.c3_decode(cuda, batch=9, num_heads=64, kv_heads=8, head_dim=64,
                               block_size=16, pool_blocks=2048, ctx_lo=1, ctx_hi=3000, seed=5)
    g = torch.Generator().manual_seed(9)
    sinks = (2 * torch.randn(64, generator=g)).to(cuda)
    ref = oracle_decode(case, window_left=window_left, sinks=sinks)
    for splits in (0, 4):
        b, hq, d = case.q.shape
        plan = ops.paged_decode_plan(b, hq, 8, d, case.max_seq_len, splits)
        ws = torch.zeros(max(1, plan.workspace_bytes), dtype=torch.uint8, device=cuda)
        out = torch.full_like(case.q, float("nan"))
        ops.paged_decode(out, case.q, case.k_cache, case.v_cache, case.block_tables,
                         case.ctx_lens, case.scale, plan.part_tokens, plan.max_parts, ws,
                         window_left=window_left, sinks=sinks)
        torch.cuda.synchronize()
        assert_close(f32(out), ref, BF16_TOL, BF16_TOL, f"window {window_left} splits {splits}")


@pytest.mark.parametrize("label,hq,hk,d", [SHAPES[0], SHAPES[1], SHAPES[3], SHAPES[5]])
@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_fused_store_decode_shapes(cuda, label, hq, hk, d, kv_dtype):
    """The fused store + decode launch equals store_kvcache then paged_decode bit for bit
    (caches and output); with groups above 16 only the kv head's first column block
    writes the row, the others read it from registers."""
    _flush(f"fused shape {label} {kv_dtype}")
    if kv_dtype == torch.bfloat16:
        case = workloads.c3_decode(cuda, batch=12, num_heads=hq, kv_heads=hk, head_dim=d,
                                   block_size=64, pool_blocks=1024, ctx_lo=1, ctx_hi=2000,
                                   seed=31 + d)
    else:
        case = workloads.c5_fp8_decode(cuda, num_heads=hq, kv_heads=hk, head_dim=d,
                                       block_size=64, ctx_lens=[1, 63, 64, 65, 900, 2000],
                                       seed=32 + d)
    rows = workloads.decode_step_rows(case)
    for splits in (0, 3):
        b, _, _ = case.q.shape
        plan = ops.paged_decode_plan(b, hq, hk, d, case.max_seq_len, splits)
        ws = torch.zeros(max(1, plan.workspace_bytes), dtype=torch.uint8, device=cuda)
        kc, vc = case.k_cache.clone(), case.v_cache.clone()
        ops.store_kvcache(rows.key, rows.value, kc, vc, rows.slot_mapping)
        sep = torch.full_like(case.q, float("nan"))
        ops.paged_decode(sep, case.q, kc, vc, case.block_tables, case.ctx_lens, case.scale,
                         plan.part_tokens, plan.max_parts, ws, case.k_scale, case.v_scale)
        kf, vf = case.k_cache.clone(), case.v_cache.clone()
        fused = torch.full_like(case.q, float("nan"))
        ops.store_paged_decode(fused, case.q, rows.key, rows.value, kf, vf, rows.slot_mapping,
                               case.block_tables, case.ctx_lens, case.scale, plan.part_tokens,
                               plan.max_parts, ws, case.k_scale, case.v_scale)
        torch.cuda.synchronize()
        raw = (lambda t: t.view(torch.uint8)) if kv_dtype != torch.bfloat16 else (lambda t: t)
        assert torch.equal(fused, sep), f"{label} splits={splits}: output"
        assert torch.equal(raw(kf), raw(kc)) and torch.equal(raw(vf), raw(vc)), \
            f"{label} splits={splits}: caches"
        tol = BF16_TOL if kv_dtype == torch.bfloat16 else FP8_TOL
        case_after = workloads.DecodeCase(case.q, kc, vc, case.block_tables, case.ctx_lens,
                                          case.scale, case.k_scale, case.v_scale)
        assert_close(f32(fused), oracle_decode(case_after), tol, tol, f"{label} vs oracle")


def test_candidate_decode_d256_and_gqa32(cuda):
    """FlashAttnDecode (the drop-in class) at head_dim 256 and at a group of 32."""
    from fastkernels_amd.candidate.L1.flash_attn_decode import FlashAttnDecode

    for hq, hk, d in ((16, 2, 256), (64, 2, 128)):
        case = workloads.c3_decode(cuda, batch=5, num_heads=hq, kv_heads=hk, head_dim=d,
                                   pool_blocks=256, ctx_lo=1, ctx_hi=4000, seed=hq + d)
        mod = FlashAttnDecode(hq, hk, d)
        out = mod(case.q, case.k_cache, case.v_cache, cache_seqlens=case.ctx_lens,
                  block_table=case.block_tables, max_seq_len=case.max_seq_len,
                  softmax_scale=case.scale)
        torch.cuda.synchronize()
        assert_close(f32(out), oracle_decode(case), BF16_TOL, BF16_TOL, f"candidate {hq}/{hk}/{d}")
