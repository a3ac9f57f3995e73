"""HIP-graph capture of a decode step built from the candidate classes.

The reference engine replays each decode step as a captured graph
(fastkernels/infra/engine.py:5386-5428, capture at :6702).  The kernels here
allocate nothing and never synchronise, so the step (add+RMSNorm -> rotary ->
store_kvcache -> paged decode -> SiLU-and-mul) must capture and replay.  New
inputs are copied into the static buffers between replays (as the engine's
graph_vars), with eager work in between, and every replay is checked against
an eager run of the same step on the same inputs.
"""
from __future__ import annotations

import pytest
import torch

from fastkernels_amd import workloads

pytestmark = pytest.mark.gpu


def _step(mods, bufs):
    norm, rope, store, attn, act = mods
    h, r = norm(bufs["hidden"], bufs["residual"])
    qkv = bufs["qkv"]
    t, hq, hk, d = bufs["dims"]
    q, k, v = qkv[:, :hq * d], qkv[:, hq * d:(hq + hk) * d], qkv[:, (hq + hk) * d:]
    rope(bufs["positions"], q, k)
    store(k.view(t, hk, d), v.view(t, hk, d), bufs["k_cache"], bufs["v_cache"], bufs["slots"])
    o = attn(q.view(t, hq, d), bufs["k_cache"], bufs["v_cache"], cache_seqlens=bufs["ctx"],
             block_table=bufs["bt"], softmax_scale=d ** -0.5, max_seq_len=bufs["max_seq_len"])
    y = act(bufs["gate_up"])
    return h, r, o, y


def test_decode_step_graph_capture_and_replay(cuda):
    from fastkernels_amd.candidate.L1.flash_attn_decode import FlashAttnDecode
    from fastkernels_amd.candidate.L1.rms_norm import RMSNorm
    from fastkernels_amd.candidate.L1.rotary_emb import RotaryEmbedding
    from fastkernels_amd.candidate.L1.silu_and_mul import SiluAndMul
    from fastkernels_amd.candidate.L1.store_kvcache import StoreKVCache

    t, hq, hk, d, hidden, inter = 32, 32, 8, 128, 4096, 1024
    cases = [workloads.c4_chain(cuda, tokens=t, inter=inter, pool_blocks=512, ctx_lo=16,
                                ctx_hi=3000, seed=300 + i) for i in range(3)]
    norm = RMSNorm(hidden).to(cuda)
    norm.weight.data.copy_(cases[0].norm_weight.float())
    norm = norm.to(torch.bfloat16)
    mods = (norm, RotaryEmbedding(d, 4096, 1e6).to(cuda), StoreKVCache(),
            FlashAttnDecode(hq, hk, d, page_size=256), SiluAndMul())
    c0 = cases[0]
    static = dict(hidden=c0.hidden.clone(), residual=c0.residual.clone(), qkv=c0.qkv.clone(),
                  positions=c0.positions.clone(), gate_up=c0.gate_up.clone(),
                  k_cache=c0.decode.k_cache.clone(), v_cache=c0.decode.v_cache.clone(),
                  slots=c0.slot_mapping.clone(), ctx=c0.decode.ctx_lens.clone(),
                  bt=torch.full((t, 16), -1, dtype=torch.int32, device=cuda),
                  dims=(t, hq, hk, d), max_seq_len=4096)
    mods[3].preallocate(t, cuda)

    def load(case):
        for key, src in (("hidden", case.hidden), ("residual", case.residual), ("qkv", case.qkv),
                         ("positions", case.positions), ("gate_up", case.gate_up),
                         ("k_cache", case.decode.k_cache), ("v_cache", case.decode.v_cache),
                         ("slots", case.slot_mapping), ("ctx", case.decode.ctx_lens)):
            static[key].copy_(src)
        bt = case.decode.block_tables  # widths differ per case: pad with -1 to the static 16
        static["bt"].fill_(-1)
        static["bt"][:, :bt.shape[1]].copy_(bt)

    # Warm up on a side stream, as torch requires before capture.
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        load(c0)
        _step(mods, static)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()

    load(c0)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = _step(mods, static)
    torch.cuda.synchronize()

    for i, case in enumerate(cases + cases[:1]):
        # eager reference on a private copy of the same inputs
        load(case)
        eager_bufs = {k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in static.items()}
        eager = [o.clone() for o in _step(mods, eager_bufs)]
        torch.cuda.synchronize()
        load(case)
        graph.replay()
        torch.cuda.synchronize()
        for name, got, ref in zip(("hidden", "residual", "attn", "act"), outs, eager):
            assert torch.equal(got, ref), f"replay {i}: {name} differs from eager"
        kflat = static["k_cache"].view(-1, hk * d)
        assert torch.equal(kflat[static["slots"]], eager_bufs["k_cache"].view(-1, hk * d)[static["slots"]])


def test_fused_store_decode_graph_capture_and_replay(cuda):
    """FlashAttnDecode.forward_store (store + decode in one launch) captured once and
    replayed on new decode-step inputs; every replay equals an eager run."""
    from fastkernels_amd.candidate.L1.flash_attn_decode import FlashAttnDecode

    b, bw = 48, 16
    cases = [workloads.c3_decode(cuda, batch=b, pool_blocks=768, ctx_lo=1, ctx_hi=4000,
                                 seed=500 + i) for i in range(3)]
    steps = [workloads.decode_step_rows(c, seed=600 + i) for i, c in enumerate(cases)]
    attn = FlashAttnDecode(32, 8, 128, page_size=256)
    attn.preallocate(b, cuda)
    c0, s0 = cases[0], steps[0]
    static = dict(q=c0.q.clone(), key=s0.key.clone(), value=s0.value.clone(),
                  k_cache=c0.k_cache.clone(), v_cache=c0.v_cache.clone(),
                  slots=s0.slot_mapping.clone(), ctx=c0.ctx_lens.clone(),
                  bt=torch.full((b, bw), -1, dtype=torch.int32, device=cuda))

    def load(case, step):
        for key, src in (("q", case.q), ("key", step.key), ("value", step.value),
                         ("k_cache", case.k_cache), ("v_cache", case.v_cache),
                         ("slots", step.slot_mapping), ("ctx", case.ctx_lens)):
            static[key].copy_(src)
        static["bt"].fill_(-1)
        static["bt"][:, :case.block_tables.shape[1]].copy_(case.block_tables)

    def run(bufs):
        return attn.forward_store(bufs["q"], bufs["key"], bufs["value"], bufs["k_cache"],
                                  bufs["v_cache"], bufs["slots"], cache_seqlens=bufs["ctx"],
                                  block_table=bufs["bt"], softmax_scale=128 ** -0.5,
                                  max_seq_len=4096)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        load(c0, s0)
        run(static)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    load(c0, s0)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = run(static)
    torch.cuda.synchronize()
    for i, (case, step) in enumerate(list(zip(cases, steps)) + [(c0, s0)]):
        load(case, step)
        eager_bufs = {k: v.clone() for k, v in static.items()}
        eager = run(eager_bufs).clone()
        torch.cuda.synchronize()
        load(case, step)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}: output differs from eager"
        assert torch.equal(static["k_cache"], eager_bufs["k_cache"]), f"replay {i}: k_cache"
        assert torch.equal(static["v_cache"], eager_bufs["v_cache"]), f"replay {i}: v_cache"


def test_prefill_merge_prologue_graph_capture_and_replay(cuda):
    """The other allocation-free entry points under one captured graph: the q/k
    norm + rotary + store prologue, paged prefill over the cache it wrote, and an
    LSE merge.  Replayed on new inputs; every replay equals an eager run."""
    from fastkernels_amd import ops

    t, hq, hk, d, bs = 64, 32, 8, 128, 16
    g = torch.Generator().manual_seed(700)

    def inputs(seed):
        gg = torch.Generator().manual_seed(seed)
        return dict(
            qkv=torch.randn(t, (hq + 2 * hk) * d, generator=gg).bfloat16().to(cuda),
            pos=torch.arange(t).to(cuda),
            po=torch.randn(t, hq, d, generator=gg).bfloat16().to(cuda),
            pl=torch.randn(hq, t, generator=gg).to(cuda),
            sl=torch.randn(hq, t, generator=gg).to(cuda))

    kc0 = torch.randn(8, bs, hk, d, generator=g).bfloat16().to(cuda)
    vc0 = torch.randn(8, bs, hk, d, generator=g).bfloat16().to(cuda)
    bt = torch.arange(8, dtype=torch.int32, device=cuda).view(1, 8)
    slots = torch.arange(t, dtype=torch.int64, device=cuda)   # positions 0..63 of sequence 0
    cu_q = torch.tensor([0, t], dtype=torch.int32, device=cuda)
    cu_k = torch.tensor([0, t], dtype=torch.int32, device=cuda)
    inv = 1.0 / (1e6 ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    ang = torch.outer(torch.arange(4096, dtype=torch.float32), inv)
    cache = torch.cat((ang.cos(), ang.sin()), -1).to(cuda)
    qw = torch.ones(d, dtype=torch.bfloat16, device=cuda)
    kw = qw.clone()

    static = inputs(701)
    static.update(kc=kc0.clone(), vc=vc0.clone(), out=torch.empty(t, hq, d, dtype=torch.bfloat16,
                                                                 device=cuda),
                  mo=torch.empty(t, hq, d, dtype=torch.bfloat16, device=cuda),
                  ml=torch.empty(hq, t, device=cuda))

    def step(bufs):
        qkv = bufs["qkv"]
        q, k, v = qkv[:, :hq * d], qkv[:, hq * d:(hq + hk) * d], qkv[:, (hq + hk) * d:]
        ops.qk_norm_rope_store(bufs["pos"], q, k, v, bufs["kc"], bufs["vc"], slots, d, cache,
                               True, qw, kw, 1e-6)
        ops.paged_prefill(bufs["out"], q.view(t, hq, d).contiguous(), bufs["kc"], bufs["vc"],
                          bt, cu_q, cu_k, t, d ** -0.5)
        ops.merge_attn_states(bufs["mo"], bufs["out"], bufs["pl"], bufs["po"], bufs["sl"],
                              bufs["ml"])
        return bufs["mo"], bufs["ml"]

    def load(src):
        for key in ("qkv", "pos", "po", "pl", "sl"):
            static[key].copy_(src[key])
        static["kc"].copy_(kc0)
        static["vc"].copy_(vc0)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(static)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    load(inputs(701))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        mo, ml = step(static)
    torch.cuda.synchronize()
    for i, seed in enumerate((702, 703, 701)):
        src = inputs(seed)
        load(src)
        eager = {k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in static.items()}
        emo, eml = (x.clone() for x in step(eager))
        torch.cuda.synchronize()
        load(src)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(mo, emo), f"replay {i}: merge output differs"
        assert torch.equal(ml, eml), f"replay {i}: merge lse differs"
        assert torch.equal(static["kc"], eager["kc"]), f"replay {i}: cache differs"
