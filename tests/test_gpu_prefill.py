"""GPU parity of paged / dense prefill attention (fk_paged_prefill, fk_varlen_prefill)
against the oracle (FlashAttnPrefill semantics, flash_attn_prefill.py:28-74, restated
from the reference's torch fallback attention_impl.py:606-652).  bf16 bar: every
element within atol = rtol = 1e-2; fp8 KV: 3e-2."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from fastkernels_amd import ops, workloads

pytestmark = pytest.mark.gpu


def _flush(msg):
    print(msg, flush=True)


def _case(cuda, q_lens, k_lens, hq=32, hk=8, bs=16, seed=70, fp8=False, extra_pages=3, d=128):
    g = torch.Generator().manual_seed(seed)
    pages = [(k + bs - 1) // bs for k in k_lens]
    nb = sum(pages) + extra_pages
    perm = torch.randperm(nb, generator=g)
    bt = torch.full((len(k_lens), max(max(pages), 1)), -1, dtype=torch.int32)
    off = 0
    for i, p in enumerate(pages):
        bt[i, :p] = perm[off:off + p].to(torch.int32)
        off += p
    cu_q = torch.tensor([0] + list(np.cumsum(q_lens)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(np.cumsum(k_lens)), dtype=torch.int32)
    q = torch.randn(int(cu_q[-1]), hq, d, generator=g).to(torch.bfloat16)
    kc = torch.randn(nb, bs, hk, d, generator=g)
    vc = torch.randn(nb, bs, hk, d, generator=g)
    ks = vs = None
    if fp8:
        ks = (0.01 + 0.09 * torch.rand(hk, generator=g)).float()
        vs = (0.01 + 0.09 * torch.rand(hk, generator=g)).float()
        kc = workloads.quantize_fp8(kc, ks)
        vc = workloads.quantize_fp8(vc, vs)
    else:
        kc, vc = kc.to(torch.bfloat16), vc.to(torch.bfloat16)
    t = lambda x: None if x is None else x.to(cuda)  # noqa: E731
    return dict(q=q.to(cuda), kc=kc.to(cuda), vc=vc.to(cuda), bt=bt.to(cuda), cu_q=cu_q.to(cuda),
                cu_k=cu_k.to(cuda), max_q=max(q_lens) if q_lens else 0,
                max_k=max(k_lens) if k_lens else 0, ks=t(ks), vs=t(vs), scale=d ** -0.5)


def _run(c, causal=True, window_left=-1, sinks=None):
    out = torch.full_like(c["q"], float("nan"))
    ops.paged_prefill(out, c["q"], c["kc"], c["vc"], c["bt"], c["cu_q"], c["cu_k"], c["max_q"],
                      c["scale"], c["ks"], c["vs"], causal, window_left, sinks,
                      max_seqlen_k=c["max_k"])
    torch.cuda.synchronize()
    return out


def _oracle(c, causal=True, window_left=-1, sinks=None):
    fp8 = c["kc"].dtype == torch.float8_e4m3fn
    kc = c["kc"].view(torch.uint8).cpu().numpy() if fp8 else c["kc"].float().cpu().numpy()
    vc = c["vc"].view(torch.uint8).cpu().numpy() if fp8 else c["vc"].float().cpu().numpy()
    return oracle.paged_prefill(c["q"].float().cpu().numpy(), kc, vc, c["bt"].cpu().numpy(),
                                c["cu_q"].cpu().numpy(), c["cu_k"].cpu().numpy(), c["scale"],
                                None if c["ks"] is None else c["ks"].cpu().numpy(),
                                None if c["vs"] is None else c["vs"].cpu().numpy(),
                                causal=causal, window_left=window_left,
                                sinks=None if sinks is None else sinks.cpu().numpy())


def _close(got, ref, tol, what):
    g = got.float().cpu().numpy()
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    err = np.abs(g - ref)
    bad = err > tol + tol * np.abs(ref)
    assert not bad.any(), f"{what}: {int(bad.sum())} elements off, max err {err.max():.3g}"


@pytest.mark.parametrize("bs", [16, 64, 256])
def test_paged_prefill_mixed_chunks(cuda, bs):
    """Whole prompts, chunked prefill over a longer context, single-token chunks and a
    chunk of 33 (a partial query block), Qwen3-8B heads (GQA 4)."""
    q_lens = [1, 5, 17, 33, 100, 64, 32]
    k_lens = [1, 5, 40, 33, 300, 1000, 47]
    _flush(f"paged prefill bs={bs}")
    c = _case(cuda, q_lens, k_lens, bs=bs, seed=71 + bs)
    _close(_run(c), _oracle(c), 1e-2, f"paged prefill bs={bs}")


@pytest.mark.parametrize("hq,hk", [(8, 8), (16, 2), (64, 8), (16, 1)])
def test_paged_prefill_gqa(cuda, hq, hk):
    _flush(f"paged prefill hq={hq} hk={hk}")
    c = _case(cuda, [20, 50], [60, 50], hq=hq, hk=hk, seed=72)
    _close(_run(c), _oracle(c), 1e-2, f"gqa {hq}/{hk}")


@pytest.mark.parametrize("hq,hk", [(16, 8), (24, 8)])
def test_paged_prefill_small_groups(cuda, hq, hk):
    """GQA 2 (each work-group's waves span two 32-query blocks of two heads) and GQA 3
    (one of the four waves has no head: it only stages K/V), over chunks that pair
    and chunks that do not."""
    _flush(f"paged prefill small groups hq={hq} hk={hk}")
    c = _case(cuda, [200, 70, 9], [200, 300, 9], hq=hq, hk=hk, bs=64, seed=75)
    _close(_run(c), _oracle(c), 1e-2, f"gqa {hq}/{hk}")


def test_paged_prefill_causal_pairing(cuda):
    """Causal chunks with few cached keys before them pair query block n-1-p with p:
    an odd block count (the middle block alone), an even one, a chunk on top of a
    shorter cached prefix (still paired), one on top of a longer prefix (not paired),
    and a block count of one."""
    _flush("paged prefill causal pairing")
    q_lens = [96, 128, 100, 100, 20]
    k_lens = [96, 128, 150, 260, 20]
    c = _case(cuda, q_lens, k_lens, bs=256, seed=76)
    _close(_run(c), _oracle(c), 1e-2, "pairing")


def test_paged_prefill_noncausal_and_empty_rows(cuda):
    """causal=False (every query sees all keys), a chunk longer than its context
    (leading rows see no key: zeros), and an empty chunk."""
    _flush("paged prefill non-causal / empty rows")
    c = _case(cuda, [10, 0, 7], [25, 9, 4], seed=73)
    _close(_run(c, causal=False), _oracle(c, causal=False), 1e-2, "non-causal")
    got = _run(c)
    _close(got, _oracle(c), 1e-2, "q_len > k_len")
    assert torch.equal(got[10:13].float(), torch.zeros_like(got[10:13].float()))


def test_paged_prefill_fp8(cuda):
    _flush("paged prefill fp8")
    c = _case(cuda, [16, 40, 1], [100, 40, 257], bs=64, seed=74, fp8=True)
    _close(_run(c), _oracle(c), 3e-2, "fp8")


def test_paged_prefill_single_token_equals_decode(cuda):
    """q_len = 1 per sequence is a decode step: same result as fk_paged_decode."""
    _flush("paged prefill == decode for one-token chunks")
    k_lens = [1, 17, 300, 1000, 4097]
    c = _case(cuda, [1] * 5, k_lens, bs=256, seed=75)
    got = _run(c)
    out = torch.empty_like(c["q"])
    part, nparts, wsb = ops.paged_decode_plan(5, 32, 8, 128, max(k_lens), 0)
    ws = torch.zeros(max(1, wsb), dtype=torch.uint8, device=cuda)
    ctx = (c["cu_k"][1:] - c["cu_k"][:-1]).to(torch.int32).contiguous()
    ops.paged_decode(out, c["q"], c["kc"], c["vc"], c["bt"], ctx, 128 ** -0.5, part, nparts, ws)
    torch.cuda.synchronize()
    _close(got, out.float().cpu().numpy(), 1e-2, "prefill vs decode")


def test_varlen_prefill_dense_strided(cuda):
    """Dense keys as strided views of a packed qkv buffer (the no-block-table path)."""
    _flush("varlen prefill dense")
    g = torch.Generator().manual_seed(76)
    q_lens, k_lens = [7, 64, 33], [7, 64, 33]
    tot = sum(q_lens)
    hq, hk = 32, 8
    qkv = torch.randn(tot, (hq + 2 * hk) * 128, generator=g).to(torch.bfloat16).to(cuda)
    q = qkv[:, :hq * 128].view(tot, hq, 128)
    k = qkv[:, hq * 128:(hq + hk) * 128].view(tot, hk, 128)
    v = qkv[:, (hq + hk) * 128:].view(tot, hk, 128)
    cu = torch.tensor([0] + list(np.cumsum(q_lens)), dtype=torch.int32, device=cuda)
    out = torch.empty(tot, hq, 128, dtype=torch.bfloat16, device=cuda)
    ops.varlen_prefill(out, q.contiguous(), k, v, cu, cu, max(q_lens), 128 ** -0.5)
    torch.cuda.synchronize()
    ref = oracle.varlen_prefill(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                v.float().cpu().numpy(), cu.cpu().numpy(), cu.cpu().numpy(),
                                128 ** -0.5)
    _close(out, ref, 1e-2, "dense varlen")


@pytest.mark.parametrize("causal,hq,hk,d,q_lens,k_lens", [
    (False, 20, 20, 64, [1500, 37], [1500, 37]),      # Whisper encoder: bidirectional, MHA, D 64
    (True, 16, 4, 128, [5, 100, 260], [5, 300, 260]),  # causal GQA, keys beyond the queries
    (False, 8, 2, 256, [64, 1], [200, 9]),
])
def test_flash_attn_varlen_candidate(cuda, causal, hq, hk, d, q_lens, k_lens):
    """FlashAttnVarlen (flash_attn_varlen.py:21-47): dense varlen attention through the
    candidate class, against oracle.varlen_prefill, with and without
    return_softmax_lse (the LSE against the oracle's within 1e-5)."""
    from fastkernels_amd.candidate.L1.flash_attn_varlen import FlashAttnVarlen
    _flush(f"FlashAttnVarlen causal={causal} hq={hq} hk={hk} d={d}")
    g = torch.Generator().manual_seed(83 + d)
    q = torch.randn(sum(q_lens), hq, d, generator=g).to(torch.bfloat16).to(cuda)
    k = torch.randn(sum(k_lens), hk, d, generator=g).to(torch.bfloat16).to(cuda)
    v = torch.randn(sum(k_lens), hk, d, generator=g).to(torch.bfloat16).to(cuda)
    cu_q = torch.tensor([0] + list(np.cumsum(q_lens)), dtype=torch.int32, device=cuda)
    cu_k = torch.tensor([0] + list(np.cumsum(k_lens)), dtype=torch.int32, device=cuda)
    m = FlashAttnVarlen()
    out = m(q, k, v, cu_q, cu_k, max(q_lens), max(k_lens), d ** -0.5, causal=causal)
    torch.cuda.synchronize()
    ref = oracle.varlen_prefill(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                v.float().cpu().numpy(), cu_q.cpu().numpy(), cu_k.cpu().numpy(),
                                d ** -0.5, causal=causal)
    _close(out, ref, 1e-2, f"FlashAttnVarlen causal={causal} d={d}")
    out2, lse = m(q, k, v, cu_q, cu_k, max(q_lens), max(k_lens), d ** -0.5, causal=causal,
                  return_softmax_lse=True)
    torch.cuda.synchronize()
    _, ref_lse = oracle.varlen_prefill(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                       v.float().cpu().numpy(), cu_q.cpu().numpy(),
                                       cu_k.cpu().numpy(), d ** -0.5, causal=causal,
                                       return_lse=True)
    assert torch.equal(out2, out)
    assert lse.shape == (hq, sum(q_lens)) and lse.dtype == torch.float32
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=1e-5, atol=1e-5)


def test_paged_prefill_qwen3_prompt_2048(cuda):
    """One 2048-token prompt at Qwen3-8B heads: against torch fp32 causal attention on
    the device (the oracle would take minutes at this size)."""
    _flush("paged prefill 2048-token prompt vs torch fp32")
    c = _case(cuda, [2048], [2048], bs=256, seed=77)
    got = _run(c)
    k = c["kc"][c["bt"][0, :8].long()].reshape(2048, 8, 128).float()
    v = c["vc"][c["bt"][0, :8].long()].reshape(2048, 8, 128).float()
    qf = c["q"].float().transpose(0, 1)                                   # [32, 2048, 128]
    kf = k.repeat_interleave(4, dim=1).transpose(0, 1).contiguous()
    vf = v.repeat_interleave(4, dim=1).transpose(0, 1).contiguous()
    ref = torch.nn.functional.scaled_dot_product_attention(qf, kf, vf, is_causal=True,
                                                           scale=128 ** -0.5)
    _close(got, ref.transpose(0, 1).cpu().numpy(), 1e-2, "2048 prompt")


@pytest.mark.parametrize("hq,hk,d", [(32, 8, 128), (16, 2, 256)])
def test_paged_prefill_fp8_prompt_2048(cuda, hq, hk, d):
    """One 2048-token prompt on fp8 pages (the key split, with the stages converted to
    bf16 in LDS), Qwen3-8B and Qwen3-Next heads: against torch fp32 causal attention on
    K / V dequantised as the reference does (float(x) * scale rounded to bf16)."""
    _flush(f"paged prefill fp8 2048-token prompt Hq={hq} Hk={hk} D={d} vs torch fp32")
    c = _case(cuda, [2048], [2048], hq=hq, hk=hk, bs=256, seed=78, fp8=True, d=d)
    got = _run(c)
    ids = c["bt"][0, :8].long()

    def deq(cache, scale):
        x = cache[ids].float().reshape(2048, hk, d) * scale.view(1, hk, 1)
        return x.to(torch.bfloat16).float().repeat_interleave(hq // hk, dim=1).transpose(0, 1)

    kf = deq(c["kc"], c["ks"]).contiguous()
    vf = deq(c["vc"], c["vs"]).contiguous()
    qf = c["q"].float().transpose(0, 1)
    ref = torch.nn.functional.scaled_dot_product_attention(qf, kf, vf, is_causal=True,
                                                           scale=d ** -0.5)
    _close(got, ref.transpose(0, 1).cpu().numpy(), 3e-2, f"fp8 2048 prompt D={d}")


@pytest.mark.parametrize("fp8", [False, True])
def test_paged_prefill_deterministic(cuda, fp8):
    """The same call repeated gives bit-identical outputs (causal chunks, masked and
    unmasked stages, paired work-groups, a window with sinks).  A tolerance check
    cannot see a kernel that reads MFMA results before they are written: its
    outputs change from run to run in the last bits."""
    _flush(f"paged prefill determinism fp8={fp8}")
    c = _case(cuda, [64, 512, 300, 1], [64, 1024, 300, 900], bs=16, seed=81, fp8=fp8)
    sinks = torch.linspace(-1.0, 2.0, 32, device=cuda)
    for kw in ({}, {"window_left": 100, "sinks": sinks}):
        first = _run(c, **kw)
        for _ in range(4):
            again = _run(c, **kw)
            assert torch.equal(again, first), f"prefill output changed between calls ({kw.keys()})"


def test_flash_attn_prefill_candidate(cuda):
    from fastkernels_amd.candidate.L1.flash_attn_prefill import FlashAttnPrefill
    _flush("FlashAttnPrefill candidate (paged)")
    c = _case(cuda, [12, 40], [50, 40], bs=16, seed=78)
    m = FlashAttnPrefill(32, 8, 128)
    out = m(c["q"], c["kc"], c["vc"], cu_seqlens_q=c["cu_q"], cu_seqlens_k=c["cu_k"],
            max_seqlen_q=40, max_seqlen_k=50, softmax_scale=128 ** -0.5, causal=True,
            block_table=c["bt"])
    torch.cuda.synchronize()
    _close(out, _oracle(c), 1e-2, "candidate")
    out = m(c["q"], c["kc"], c["vc"], c["cu_q"], c["cu_k"], 40, 50, block_table=c["bt"],
            window_size=(20, 0))
    torch.cuda.synchronize()
    _close(out, _oracle(c, window_left=20), 1e-2, "candidate, window (20, 0)")


def test_mixed_batch_like_forward_mixed(cuda):
    """Attention._forward_mixed (attention_impl.py:682-731): the first np_ tokens are
    prefill chunks (FlashAttnPrefill with a block table), the rest decode tokens
    (FlashAttnDecode), written into one output; each part against the oracle."""
    from fastkernels_amd.candidate.L1.flash_attn_decode import FlashAttnDecode
    from fastkernels_amd.candidate.L1.flash_attn_prefill import FlashAttnPrefill
    _flush("mixed prefill + decode batch")
    q_lens, k_lens = [37, 16], [37, 200]          # prefill chunks
    dec_lens = [5, 300, 1024, 77]                 # decode contexts
    c = _case(cuda, q_lens + [1] * 4, k_lens + dec_lens, bs=64, seed=79)
    np_ = sum(q_lens)
    q = c["q"]
    out = torch.empty_like(q)
    pre = FlashAttnPrefill(32, 8, 128)
    dec = FlashAttnDecode(32, 8, 128, page_size=64)
    cu_q = c["cu_q"][:3].contiguous()
    cu_k = c["cu_k"][:3].contiguous()
    out[:np_] = pre(q[:np_], c["kc"], c["vc"], cu_seqlens_q=cu_q, cu_seqlens_k=cu_k,
                    max_seqlen_q=max(q_lens), max_seqlen_k=max(k_lens), softmax_scale=128 ** -0.5,
                    causal=True, block_table=c["bt"][:2])
    ctx = torch.tensor(dec_lens, dtype=torch.int32, device=cuda)
    out[np_:] = dec(q[np_:], c["kc"], c["vc"], cache_seqlens=ctx, block_table=c["bt"][2:],
                    softmax_scale=128 ** -0.5, causal=True, max_seq_len=max(dec_lens))
    torch.cuda.synchronize()
    _close(out, _oracle(c), 1e-2, "mixed batch")


@pytest.mark.parametrize("window_left", [0, 7, 31, 32, 100, 511, 4000])
@pytest.mark.parametrize("fp8", [False, True])
def test_paged_prefill_sliding_window_and_sinks(cuda, window_left, fp8):
    """Causal sliding window (window_size = (window_left, 0)) across tile (16), stage
    (32) and page edges, in whole prompts, chunks over a longer context and a
    one-token chunk, with and without attention sinks; GQA 4 (Qwen3-8B heads)."""
    _flush(f"prefill window={window_left} fp8={fp8}")
    q_lens = [1, 17, 100, 257, 64]
    k_lens = [40, 17, 612, 257, 1000]
    c = _case(cuda, q_lens, k_lens, bs=64, seed=90 + window_left, fp8=fp8)
    g = torch.Generator().manual_seed(91)
    sinks = (2 * torch.randn(32, generator=g)).float().to(cuda)
    tol = 3e-2 if fp8 else 1e-2
    for sk in (None, sinks):
        _close(_run(c, True, window_left, sk), _oracle(c, True, window_left, sk), tol,
               f"window={window_left} sinks={sk is not None}")


def test_prefill_window_sinks_dense_and_candidate(cuda):
    """The dense path (fk_varlen_prefill) with a window and sinks, and FlashAttnPrefill
    as Attention._forward_pure calls it (window_size, s_aux in the model dtype;
    attention_impl.py:401-434), paged and dense; a window without causal is refused."""
    from fastkernels_amd.candidate.L1.flash_attn_prefill import FlashAttnPrefill

    q_lens, k_lens = [33, 200, 5], [33, 200, 5]
    c = _case(cuda, q_lens, k_lens, hq=16, hk=4, bs=16, seed=92)
    g = torch.Generator().manual_seed(93)
    s_aux = (2 * torch.randn(16, generator=g)).to(torch.bfloat16).to(cuda)
    ref = _oracle(c, True, 63, s_aux.float())
    # dense keys: the sequences' pages gathered into [total_k, Hk, D]
    bt, cu_k = c["bt"].cpu(), c["cu_k"].cpu()
    rows = torch.cat([torch.arange(int(bt[i, t // 16]) * 16 + t % 16, int(bt[i, t // 16]) * 16
                                   + t % 16 + 1) for i, n in enumerate(k_lens) for t in range(n)])
    k = c["kc"].view(-1, 4, 128)[rows.to(cuda)]
    v = c["vc"].view(-1, 4, 128)[rows.to(cuda)]
    out = torch.full_like(c["q"], float("nan"))
    ops.varlen_prefill(out, c["q"], k, v, c["cu_q"], c["cu_k"], c["max_q"], 128 ** -0.5, True,
                       63, s_aux.float())
    torch.cuda.synchronize()
    _close(out, ref, 1e-2, "dense window + sinks")
    mod = FlashAttnPrefill(16, 4, 128)
    kw = dict(softmax_scale=128 ** -0.5, causal=True, window_size=(63, 0), s_aux=s_aux)
    got = mod(c["q"], c["kc"], c["vc"], cu_seqlens_q=c["cu_q"], cu_seqlens_k=c["cu_k"],
              max_seqlen_q=c["max_q"], max_seqlen_k=max(k_lens), block_table=c["bt"], **kw)
    _close(got, ref, 1e-2, "candidate paged")
    got = mod(c["q"], k.reshape(-1, 4 * 128), v.reshape(-1, 4 * 128), cu_seqlens_q=c["cu_q"],
              cu_seqlens_k=c["cu_k"], max_seqlen_q=c["max_q"], max_seqlen_k=max(k_lens), **kw)
    _close(got, ref, 1e-2, "candidate dense")
    with pytest.raises(NotImplementedError):
        mod(c["q"], c["kc"], c["vc"], cu_seqlens_q=c["cu_q"], cu_seqlens_k=c["cu_k"],
            max_seqlen_q=c["max_q"], max_seqlen_k=max(k_lens), block_table=c["bt"],
            causal=False, window_size=(63, 0))


# ---------------------------------------------------------------------------
# Head sizes 64 and 256, and query groups above 16 (the shapes the reference builds
# FlashAttnPrefill with besides Qwen3-8B's: Qwen3-Next 16/2/256,
# L2/qwen3_next_attention.py:148-150; Whisper's self-attention, MHA at 64,
# L2/whisper_attention.py:185-190).
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("hq,hk,d", [(16, 2, 256), (20, 20, 64), (64, 8, 64), (64, 2, 128),
                                     (40, 1, 256), (71, 1, 64)])
def test_paged_prefill_head_sizes_and_groups(cuda, hq, hk, d):
    _flush(f"paged prefill hq={hq} hk={hk} d={d}")
    c = _case(cuda, [1, 33, 100, 64], [1, 33, 300, 1000], hq=hq, hk=hk, bs=64, d=d,
              seed=hq + hk + d)
    _close(_run(c), _oracle(c), 1e-2, f"{hq}/{hk}/{d}")
    _close(_run(c, causal=False), _oracle(c, causal=False), 1e-2, f"{hq}/{hk}/{d} non-causal")


@pytest.mark.parametrize("d", [64, 256])
def test_paged_prefill_head_sizes_fp8(cuda, d):
    _flush(f"paged prefill fp8 d={d}")
    c = _case(cuda, [16, 40, 1], [100, 40, 257], hq=16, hk=2, bs=64, seed=74 + d, fp8=True, d=d)
    _close(_run(c), _oracle(c), 3e-2, f"fp8 d={d}")


@pytest.mark.parametrize("d", [64, 256])
def test_paged_prefill_head_sizes_window_and_sinks(cuda, d):
    """A gpt-oss-like layer (64 query heads, 8 kv heads, a 128-token window, sinks)
    at head size 64, and the same at 256."""
    _flush(f"paged prefill window+sinks d={d}")
    c = _case(cuda, [300, 7], [500, 200], hq=64, hk=8, bs=16, seed=80 + d, d=d)
    g = torch.Generator().manual_seed(81)
    sinks = (2 * torch.randn(64, generator=g)).to(cuda)
    _close(_run(c, window_left=127, sinks=sinks), _oracle(c, window_left=127, sinks=sinks), 1e-2,
           f"window+sinks d={d}")


@pytest.mark.parametrize("hq,hk,d", [(20, 20, 64), (16, 2, 256)])
def test_varlen_prefill_head_sizes(cuda, hq, hk, d):
    """Dense keys (no block table) at head sizes 64 and 256: Whisper's encoder
    self-attention is this path, non-causal over the whole segment."""
    _flush(f"varlen prefill hq={hq} hk={hk} d={d}")
    g = torch.Generator().manual_seed(90 + d)
    q_lens, k_lens = [50, 1500, 3], [50, 1500, 9]
    cu_q = torch.tensor([0] + list(np.cumsum(q_lens)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(np.cumsum(k_lens)), dtype=torch.int32)
    q = torch.randn(int(cu_q[-1]), hq, d, generator=g).to(torch.bfloat16).to(cuda)
    kv = torch.randn(int(cu_k[-1]), 2, hk, d, generator=g).to(torch.bfloat16).to(cuda)
    key, value = kv[:, 0], kv[:, 1]  # strided views, rows 2 * hk * d apart
    for causal in (False, True):
        out = torch.full_like(q, float("nan"))
        ops.varlen_prefill(out, q, key, value, cu_q.to(cuda), cu_k.to(cuda), max(q_lens),
                           d ** -0.5, causal)
        torch.cuda.synchronize()
        ref = oracle.varlen_prefill(q.float().cpu().numpy(), key.float().cpu().numpy(),
                                    value.float().cpu().numpy(), cu_q.numpy(), cu_k.numpy(),
                                    d ** -0.5, causal)
        _close(out, ref, 1e-2, f"varlen {hq}/{hk}/{d} causal={causal}")


def test_candidate_prefill_head_size_256(cuda):
    """FlashAttnPrefill (the drop-in class) at Qwen3-Next's head size, paged and dense."""
    from fastkernels_amd.candidate.L1.flash_attn_prefill import FlashAttnPrefill

    c = _case(cuda, [40, 200], [40, 600], hq=16, hk=2, bs=64, d=256, seed=95)
    mod = FlashAttnPrefill(16, 2, 256)
    out = mod(c["q"], c["kc"], c["vc"], c["cu_q"], c["cu_k"], c["max_q"], 600,
              block_table=c["bt"])
    torch.cuda.synchronize()
    _close(out, _oracle(c), 1e-2, "candidate d=256")


# The kernel splits each query block's keys between two halves of an 8-wave work-group
# when the grid (sized by max_seqlen_q) would have fewer than two work-groups per CU,
# and streams them in one pass otherwise.  The same inputs with max_seqlen_q at its
# exact value and raised to 20000 (a larger bound is allowed; the extra blocks have no
# work) take the two forms.
SPLIT_CASES = [
    # (label, q_lens, k_lens, kwargs)
    ("prompt 700 (paired blocks)", [700], [700], {}),
    ("chunk 96 over 3000", [96], [3000], {}),
    ("mixed", [1, 257, 33], [900, 257, 2000], {"bs": 64}),
    ("fp8", [130, 5], [1000, 77], {"fp8": True, "bs": 64}),
    ("head 64, group 8", [300, 64], [300, 1000], {"hq": 64, "hk": 8, "d": 64}),
]


@pytest.mark.parametrize("label,q_lens,k_lens,kw", SPLIT_CASES)
def test_paged_prefill_key_split_and_single_pass(cuda, label, q_lens, k_lens, kw):
    _flush(f"prefill key split vs single pass: {label}")
    c = _case(cuda, q_lens, k_lens, seed=300 + len(label), **kw)
    tol = 3e-2 if kw.get("fp8") else 1e-2
    ref = _oracle(c)
    split = _run(c)
    whole = _run(dict(c, max_q=20000))
    _close(split, ref, tol, f"{label}: key split")
    _close(whole, ref, tol, f"{label}: single pass")
    assert torch.equal(_run(dict(c, max_q=20000)), whole), f"{label}: single pass repeat"
    assert torch.equal(_run(c), split), f"{label}: key split repeat"


@pytest.mark.parametrize("window_left", [0, 31, 200])
def test_paged_prefill_key_split_window_and_sinks(cuda, window_left):
    """Sliding window and sinks through both halves of the key split (the first
    half's stages may all lie before a query's window) and the single pass."""
    _flush(f"prefill key split window={window_left}")
    c = _case(cuda, [400, 9], [1200, 300], bs=16, seed=310 + window_left)
    g = torch.Generator().manual_seed(311)
    sinks = (2 * torch.randn(32, generator=g)).float().to(cuda)
    ref = _oracle(c, window_left=window_left, sinks=sinks)
    _close(_run(c, window_left=window_left, sinks=sinks), ref, 1e-2, "key split")
    _close(_run(dict(c, max_q=20000), window_left=window_left, sinks=sinks), ref, 1e-2,
           "single pass")


def _masked_page_reference(c, holes):
    """float64 attention with the kernel's rule for a -1 block-table entry inside a
    sequence's pages: its keys are masked (not read), causal positions unchanged;
    a query with no visible key gives a zero row.  holes: (sequence, page index)."""
    q = c["q"].double().cpu()
    kc, vc = c["kc"].double().cpu(), c["vc"].double().cpu()
    bt = c["bt"].cpu().clone()
    for b, p in holes:
        bt[b, p] = -1
    cu_q, cu_k = c["cu_q"].cpu().tolist(), c["cu_k"].cpu().tolist()
    bs, hk = kc.shape[1], kc.shape[2]
    hq = q.shape[1]
    out = torch.zeros(q.shape, dtype=torch.float64)
    for i in range(len(cu_q) - 1):
        q_len, k_len = cu_q[i + 1] - cu_q[i], cu_k[i + 1] - cu_k[i]
        if q_len == 0:
            continue
        pages = bt[i, :(k_len + bs - 1) // bs]
        ok_page = pages >= 0
        ks = kc[pages.clamp(min=0).long()].reshape(-1, hk, kc.shape[-1])[:k_len]
        vs = vc[pages.clamp(min=0).long()].reshape(-1, hk, vc.shape[-1])[:k_len]
        key_ok = ok_page.repeat_interleave(bs)[:k_len]
        pos = torch.arange(k_len - q_len, k_len)
        vis = (torch.arange(k_len)[None, :] <= pos[:, None]) & key_ok[None, :]
        qi = q[cu_q[i]:cu_q[i + 1]]
        kk = ks.repeat_interleave(hq // hk, dim=1)
        vv = vs.repeat_interleave(hq // hk, dim=1)
        s = torch.einsum("qhd,khd->hqk", qi, kk) * c["scale"]
        s = s.masked_fill(~vis[None], float("-inf"))
        p = torch.softmax(s, dim=-1).nan_to_num(0.0)
        out[cu_q[i]:cu_q[i + 1]] = torch.einsum("hqk,khd->qhd", p, vv)
    return out.numpy(), bt


@pytest.mark.parametrize("label,q_lens,k_lens,bs,holes", [
    # a chunk over a longer cache: the hole lies in the stages every query sees in full
    ("chunk, 16-token pages", [300], [700], 16, [(0, 5), (0, 30)]),
    # a 2048-token prompt: paired blocks with the key split; 256-token pages
    ("prompt 2048, 256-token pages", [2048], [2048], 256, [(0, 2)]),
    # four chunks with holes at different places, 64-token pages
    ("4 chunks, 64-token pages", [128] * 4, [1024] * 4, 64, [(0, 1), (1, 7), (2, 15), (3, 0)]),
    # one chunk over a long cache: the work-group key split's parts
    ("chunk over 8192, key-split parts", [512], [8192], 256, [(0, 10), (0, 29)]),
])
def test_paged_prefill_masked_pages(cuda, label, q_lens, k_lens, bs, holes):
    """A -1 block-table entry inside a sequence's pages masks that page's keys (the
    kernel reads page 0 in its place and discards it).  The reference leaves such a
    table undefined (its torch path indexes block -1), so the check is against the
    kernel's own rule, restated in float64 torch."""
    _flush(f"masked pages: {label}")
    c = _case(cuda, q_lens, k_lens, bs=bs, seed=91)
    ref, bt = _masked_page_reference(c, holes)
    c["bt"] = bt.to(cuda)
    got = _run(c)
    _close(got, ref, 1e-2, f"masked pages, {label}")
    assert torch.equal(_run(c), got), f"masked pages, {label}: repeat"
