"""Randomised parity sweep: decode and prefill over seeded combinations of the
options the targeted tests cover one or two at a time (head size, GQA group,
page size, bf16 / fp8 pages, window, sinks, schedule, causal / dense), each
against the CPU oracle at the same bars (bf16 atol = rtol = 1e-2, fp8 3e-2).

Sizes stay small so that the numpy oracle finishes in seconds; every case prints
its parameters before it runs.  FK_RANDOM_SCALE=k runs k times as many cases.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import oracle
from fastkernels_amd import ops, workloads

pytestmark = pytest.mark.gpu

# Case counts; FK_RANDOM_SCALE multiplies them for a wider sweep (seeds stay fixed per case).
_SCALE = max(1, int(os.environ.get("FK_RANDOM_SCALE", "1")))
N_DECODE = 120 * _SCALE
N_PREFILL = 80 * _SCALE


def _close(got, ref, tol, what):
    g = got.float().cpu().numpy().astype(np.float64)
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    err = np.abs(g - ref)
    bad = err > tol + tol * np.abs(ref)
    assert not bad.any(), f"{what}: {int(bad.sum())}/{bad.size} off, max err {err.max():.3g}"


def _decode_params(i):
    rng = np.random.default_rng(1000 + i)
    d = int(rng.choice([64, 128, 256]))
    hk = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([1, 2, 4, 5, 8, 16, 20]))
    bs = int(rng.choice([16, 32, 64, 256]))
    b = int(rng.integers(1, 9))
    long_ctx = rng.random() < 0.3
    ctx = rng.integers(0, 6000 if long_ctx else 700, b).tolist()
    fp8 = bool(rng.random() < 0.35)
    window = int(rng.choice([-1, -1, 0, 17, 300]))
    sinks = bool(rng.random() < 0.3)
    splits = int(rng.choice([0, 0, 0, 3, 16]))
    return dict(d=d, hk=hk, hq=hk * group, bs=bs, ctx=ctx, fp8=fp8, window=window,
                sinks=sinks, splits=splits, seed=2000 + i)


@pytest.mark.parametrize("i", range(N_DECODE))
def test_random_decode(cuda, i):
    p = _decode_params(i)
    print(f"random decode {i}: {p}", flush=True)
    pool = sum((n + p["bs"] - 1) // p["bs"] for n in p["ctx"]) + 2
    if p["fp8"]:
        case = workloads.c5_fp8_decode(cuda, num_heads=p["hq"], kv_heads=p["hk"], head_dim=p["d"],
                                       block_size=p["bs"], pool_blocks=pool, seed=p["seed"],
                                       ctx_lens=p["ctx"])
    else:
        case = workloads.c3_decode(cuda, num_heads=p["hq"], kv_heads=p["hk"], head_dim=p["d"],
                                   block_size=p["bs"], pool_blocks=pool, seed=p["seed"],
                                   ctx_lens=p["ctx"])
    sinks = None
    if p["sinks"]:
        g = torch.Generator().manual_seed(p["seed"])
        sinks = (2 * torch.randn(p["hq"], generator=g)).float().to(cuda)
    b, hq, d = case.q.shape
    part, nparts, wsb = ops.paged_decode_plan(b, hq, p["hk"], d, max(1, case.max_seq_len),
                                              p["splits"])
    ws = torch.zeros(max(1, wsb), dtype=torch.uint8, device=cuda)
    out = torch.full_like(case.q, float("nan"))
    ops.paged_decode(out, case.q, case.k_cache, case.v_cache, case.block_tables, case.ctx_lens,
                     case.scale, part, nparts, ws, case.k_scale, case.v_scale, p["window"], sinks)
    torch.cuda.synchronize()
    bt = case.block_tables.cpu().numpy()
    ctx = case.ctx_lens.cpu().numpy()
    if p["fp8"]:
        kc = case.k_cache.view(torch.uint8).cpu().numpy()
        vc = case.v_cache.view(torch.uint8).cpu().numpy()
    else:
        kc, vc = case.k_cache.float().cpu().numpy(), case.v_cache.float().cpu().numpy()
    ref = oracle.paged_decode(
        case.q.float().cpu().numpy(), kc, vc, bt, ctx, case.scale,
        None if case.k_scale is None else case.k_scale.cpu().numpy(),
        None if case.v_scale is None else case.v_scale.cpu().numpy(),
        window_left=p["window"], sinks=None if sinks is None else sinks.cpu().numpy())
    _close(out, ref, 3e-2 if p["fp8"] else 1e-2, f"random decode {i} {p}")
    for k, n in enumerate(p["ctx"]):
        if n == 0:
            assert not out[k].float().abs().sum().item(), f"random decode {i}: empty row {k}"


def _prefill_params(i):
    rng = np.random.default_rng(3000 + i)
    d = int(rng.choice([64, 128, 256]))
    hk = int(rng.choice([1, 2, 8]))
    group = int(rng.choice([1, 4, 5, 8]))
    bs = int(rng.choice([16, 64, 256]))
    n = int(rng.integers(1, 5))
    q_lens, k_lens = [], []
    for _ in range(n):
        ql = int(rng.integers(1, 300))
        kl = ql + int(rng.choice([0, 0, int(rng.integers(1, 900))]))
        q_lens.append(ql)
        k_lens.append(kl)
    causal = bool(rng.random() < 0.8)
    window = int(rng.choice([-1, -1, -1, 0, 31, 200])) if causal else -1
    fp8 = bool(rng.random() < 0.3)
    sinks = bool(rng.random() < 0.3)
    dense = bool(rng.random() < 0.25) and not fp8
    return dict(d=d, hk=hk, hq=hk * group, bs=bs, q_lens=q_lens, k_lens=k_lens, causal=causal,
                window=window, fp8=fp8, sinks=sinks, dense=dense, seed=4000 + i)


def _prefill_params_long(i):
    """Chunks over long caches (the launches that split each block's keys over
    work-groups, with the key split or with 4-wave work-groups), heads kept few so that
    the oracle stays within seconds."""
    rng = np.random.default_rng(5000 + i)
    d = int(rng.choice([64, 128]))
    hk, group = [(2, 1), (2, 2), (2, 4), (4, 1), (4, 2), (4, 4), (8, 1), (8, 2)][
        int(rng.integers(0, 8))]
    bs = int(rng.choice([16, 64, 256]))
    n = int(rng.integers(1, 4))
    q_lens = [int(rng.integers(200, 513)) for _ in range(n)]
    k_lens = [int(rng.integers(2048, 8193)) for _ in range(n)]
    causal = bool(rng.random() < 0.8)
    window = int(rng.choice([-1, -1, -1, -1, 300, 2000])) if causal else -1
    fp8 = bool(rng.random() < 0.3)
    sinks = bool(rng.random() < 0.3)
    dense = bool(rng.random() < 0.25) and not fp8
    return dict(d=d, hk=hk, hq=hk * group, bs=bs, q_lens=q_lens, k_lens=k_lens, causal=causal,
                window=window, fp8=fp8, sinks=sinks, dense=dense, seed=6000 + i)


N_PREFILL_LONG = 16 * _SCALE


@pytest.mark.parametrize("i", range(N_PREFILL))
def test_random_prefill(cuda, i):
    _random_prefill(cuda, f"random prefill {i}", _prefill_params(i))


@pytest.mark.parametrize("i", range(N_PREFILL_LONG))
def test_random_prefill_long_caches(cuda, i):
    _random_prefill(cuda, f"random prefill over a long cache {i}", _prefill_params_long(i))


def _random_prefill(cuda, i, p):
    print(f"{i}: {p}", flush=True)
    g = torch.Generator().manual_seed(p["seed"])
    hq, hk, d, bs = p["hq"], p["hk"], p["d"], p["bs"]
    q_lens, k_lens = p["q_lens"], p["k_lens"]
    cu_q = torch.tensor([0] + list(np.cumsum(q_lens)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(np.cumsum(k_lens)), dtype=torch.int32)
    q = torch.randn(int(cu_q[-1]), hq, d, generator=g).to(torch.bfloat16)
    sinks = (2 * torch.randn(hq, generator=g)).float() if p["sinks"] else None
    scale = d ** -0.5
    out = torch.full((int(cu_q[-1]), hq, d), float("nan"), dtype=torch.bfloat16, device=cuda)
    if p["dense"]:
        k = torch.randn(int(cu_k[-1]), hk, d, generator=g).to(torch.bfloat16)
        v = torch.randn(int(cu_k[-1]), hk, d, generator=g).to(torch.bfloat16)
        ops.varlen_prefill(out, q.to(cuda), k.to(cuda), v.to(cuda), cu_q.to(cuda), cu_k.to(cuda),
                           max(q_lens), scale, p["causal"], p["window"],
                           None if sinks is None else sinks.to(cuda), max(k_lens))
        torch.cuda.synchronize()
        ref = oracle.varlen_prefill(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                    cu_q.numpy(), cu_k.numpy(), scale, causal=p["causal"],
                                    window_left=p["window"],
                                    sinks=None if sinks is None else sinks.numpy())
        _close(out, ref, 1e-2, f"{i} {p}")
        return
    pages = [(kl + bs - 1) // bs for kl in k_lens]
    nb = sum(pages) + 2
    perm = torch.randperm(nb, generator=g)
    bt = torch.full((len(k_lens), max(pages)), -1, dtype=torch.int32)
    off = 0
    for j, pg in enumerate(pages):
        bt[j, :pg] = perm[off:off + pg].to(torch.int32)
        off += pg
    kc = torch.randn(nb, bs, hk, d, generator=g)
    vc = torch.randn(nb, bs, hk, d, generator=g)
    ks = vs = None
    if p["fp8"]:
        ks = (0.01 + 0.09 * torch.rand(hk, generator=g)).float()
        vs = (0.01 + 0.09 * torch.rand(hk, generator=g)).float()
        kc, vc = workloads.quantize_fp8(kc, ks), workloads.quantize_fp8(vc, vs)
    else:
        kc, vc = kc.to(torch.bfloat16), vc.to(torch.bfloat16)
    dev = lambda x: None if x is None else x.to(cuda)  # noqa: E731
    ops.paged_prefill(out, q.to(cuda), kc.to(cuda), vc.to(cuda), bt.to(cuda), cu_q.to(cuda),
                      cu_k.to(cuda), max(q_lens), scale, dev(ks), dev(vs), p["causal"],
                      p["window"], dev(sinks), max_seqlen_k=max(k_lens))
    torch.cuda.synchronize()
    kn = kc.view(torch.uint8).numpy() if p["fp8"] else kc.float().numpy()
    vn = vc.view(torch.uint8).numpy() if p["fp8"] else vc.float().numpy()
    ref = oracle.paged_prefill(q.float().numpy(), kn, vn, bt.numpy(), cu_q.numpy(), cu_k.numpy(),
                               scale, None if ks is None else ks.numpy(),
                               None if vs is None else vs.numpy(), causal=p["causal"],
                               window_left=p["window"],
                               sinks=None if sinks is None else sinks.numpy())
    _close(out, ref, 3e-2 if p["fp8"] else 1e-2, f"{i} {p}")


N_FUSED = 40 * _SCALE


@pytest.mark.parametrize("i", range(N_FUSED))
def test_random_fused_store_decode(cuda, i):
    """store_paged_decode against store_kvcache then paged_decode on copies of the
    caches (bit for bit: output and both caches), over random decode options."""
    p = _decode_params(500 + i)
    p["ctx"] = [n + 1 for n in p["ctx"]]  # a decode step: the new token is position ctx - 1
    print(f"random fused store + decode {i}: {p}", flush=True)
    pool = sum((n + p["bs"] - 1) // p["bs"] for n in p["ctx"]) + 2
    build = workloads.c5_fp8_decode if p["fp8"] else workloads.c3_decode
    case = build(cuda, num_heads=p["hq"], kv_heads=p["hk"], head_dim=p["d"], block_size=p["bs"],
                 pool_blocks=pool, seed=p["seed"], ctx_lens=p["ctx"])
    rows = workloads.decode_step_rows(case, seed=p["seed"] + 1)
    sinks = None
    if p["sinks"]:
        g = torch.Generator().manual_seed(p["seed"])
        sinks = (2 * torch.randn(p["hq"], generator=g)).float().to(cuda)
    b, hq, d = case.q.shape
    part, nparts, wsb = ops.paged_decode_plan(b, hq, p["hk"], d, case.max_seq_len, p["splits"])
    res = []
    for fused in (False, True):
        kc, vc = case.k_cache.clone(), case.v_cache.clone()
        ws = torch.zeros(max(1, wsb), dtype=torch.uint8, device=cuda)
        out = torch.full_like(case.q, float("nan"))
        if fused:
            ops.store_paged_decode(out, case.q, rows.key, rows.value, kc, vc, rows.slot_mapping,
                                   case.block_tables, case.ctx_lens, case.scale, part, nparts,
                                   ws, case.k_scale, case.v_scale, p["window"], sinks)
        else:
            ops.store_kvcache(rows.key, rows.value, kc, vc, rows.slot_mapping)
            ops.paged_decode(out, case.q, kc, vc, case.block_tables, case.ctx_lens, case.scale,
                             part, nparts, ws, case.k_scale, case.v_scale, p["window"], sinks)
        torch.cuda.synchronize()
        res.append((out, kc, vc))
    for name, a, c in zip(("out", "k_cache", "v_cache"), res[1], res[0]):
        if a.dtype == torch.float8_e4m3fn:
            a, c = a.view(torch.uint8), c.view(torch.uint8)
        assert torch.equal(a, c), f"random fused {i} {p}: {name} differs from the two calls"
