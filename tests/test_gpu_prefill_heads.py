"""GPU parity of the prefill kernel at the head sizes and outputs the reference's other
callers need, against the oracle:

- FlashAttnVarlen's return_softmax_lse (flash_attn_varlen.py:33-46): the rows'
  log-sum-exp within rtol = atol = 1e-5 of the oracle's float64 value, -inf for rows
  with no visible key, through the key split and the single pass;
- MLA prefill (L2/mla_attention_impl.py:347-398): query / key head 192 with value head
  128, causal over new tokens and non-causal over cached-context chunks whose
  (out, lse) pairs merge_attn_states combines into the attention over all the keys;
- head sizes 32, 72, 80 and 96 (small encoders, Qwen3-VL's and Qwen2/2.5-VL's vision
  encoders, L2/vision_attention.py:32,39), dense and paged, and FlashAttnPrefill at 80.

Outputs: every element within atol = rtol = 1e-2 (bf16)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from fastkernels_amd import ops

pytestmark = pytest.mark.gpu


def _flush(msg):
    print(msg, flush=True)


def _close(got, ref, tol, what):
    g = got.float().cpu().numpy()
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    err = np.abs(g - ref)
    bad = err > tol + tol * np.abs(ref)
    assert not bad.any(), f"{what}: {int(bad.sum())} elements off, max err {err.max():.3g}"


def _lse_close(got, ref, what):
    g = got.cpu().numpy()
    assert np.array_equal(np.isneginf(g), np.isneginf(ref)), f"{what}: -inf rows differ"
    fin = np.isfinite(ref)
    assert np.isfinite(g[fin]).all(), f"{what}: non-finite lse"
    np.testing.assert_allclose(g[fin], ref[fin], rtol=1e-5, atol=1e-5, err_msg=what)


def _dense(cuda, q_lens, k_lens, hq, hk, d, dv=None, seed=0):
    dv = d if dv is None else dv
    g = torch.Generator().manual_seed(seed)
    cu_q = torch.tensor([0] + list(np.cumsum(q_lens)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(np.cumsum(k_lens)), dtype=torch.int32)
    q = torch.randn(int(cu_q[-1]), hq, d, generator=g).to(torch.bfloat16)
    k = torch.randn(int(cu_k[-1]), hk, d, generator=g).to(torch.bfloat16)
    v = torch.randn(int(cu_k[-1]), hk, dv, generator=g).to(torch.bfloat16)
    return (q.to(cuda), k.to(cuda), v.to(cuda), cu_q.to(cuda), cu_k.to(cuda))


def _run_dense(q, k, v, cu_q, cu_k, max_q, scale, causal, lse=False, max_k=0):
    out = torch.full((q.shape[0], q.shape[1], v.shape[2]), float("nan"), dtype=q.dtype,
                     device=q.device)
    lt = (torch.full((q.shape[1], q.shape[0]), float("nan"), dtype=torch.float32,
                     device=q.device) if lse else None)
    ops.varlen_prefill(out, q, k, v, cu_q, cu_k, max_q, scale, causal, max_seqlen_k=max_k,
                       lse=lt)
    torch.cuda.synchronize()
    return out, lt


def _oracle_dense(q, k, v, cu_q, cu_k, scale, causal, lse=False):
    return oracle.varlen_prefill(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                 v.float().cpu().numpy(), cu_q.cpu().numpy(), cu_k.cpu().numpy(),
                                 scale, causal=causal, return_lse=lse)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("hq,hk,d", [(32, 8, 128), (16, 16, 64), (8, 2, 256)])
def test_varlen_lse_key_split_and_single_pass(cuda, causal, hq, hk, d):
    """The LSE through the key split (max_seqlen_q exact, few work-groups) and the single
    pass (max_seqlen_q raised), with a causal chunk longer than its keys (rows with no
    visible key: lse -inf, output 0) and a one-token sequence."""
    _flush(f"varlen lse causal={causal} {hq}/{hk}/{d}")
    q_lens, k_lens = [300, 1, 70], [900, 5, 40]
    q, k, v, cu_q, cu_k = _dense(cuda, q_lens, k_lens, hq, hk, d, seed=d + causal)
    scale = d ** -0.5
    ref, ref_lse = _oracle_dense(q, k, v, cu_q, cu_k, scale, causal, lse=True)
    if causal:
        assert np.isneginf(ref_lse).any()  # the 70-query chunk over 40 keys
    for max_q in (max(q_lens), 20000):
        out, lse = _run_dense(q, k, v, cu_q, cu_k, max_q, scale, causal, lse=True,
                              max_k=max(k_lens))
        _close(out, ref, 1e-2, f"out max_q={max_q}")
        _lse_close(lse, ref_lse, f"lse max_q={max_q}")
        plain, _ = _run_dense(q, k, v, cu_q, cu_k, max_q, scale, causal, max_k=max(k_lens))
        assert torch.equal(plain, out), "the LSE variant changes the output"


def test_varlen_lse_with_sinks_and_strided_rows(cuda):
    """lse with attention sinks (the sink joins the denominator and the log-sum-exp) and an
    lse tensor wider than total_q (its row stride is honoured)."""
    _flush("varlen lse sinks")
    q, k, v, cu_q, cu_k = _dense(cuda, [40, 200], [100, 200], 16, 4, 128, seed=5)
    g = torch.Generator().manual_seed(6)
    sinks = (2 * torch.randn(16, generator=g)).float().to(cuda)
    wide = torch.full((16, 300), 7.0, dtype=torch.float32, device=cuda)
    out = torch.empty((240, 16, 128), dtype=torch.bfloat16, device=cuda)
    ops.varlen_prefill(out, q, k, v, cu_q, cu_k, 200, 128 ** -0.5, True, sinks=sinks, lse=wide)
    torch.cuda.synchronize()
    ref, ref_lse = oracle.varlen_prefill(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                         v.float().cpu().numpy(), cu_q.cpu().numpy(),
                                         cu_k.cpu().numpy(), 128 ** -0.5, True,
                                         sinks=sinks.cpu().numpy(), return_lse=True)
    _close(out, ref, 1e-2, "sinks out")
    _lse_close(wide[:, :240], ref_lse, "sinks lse")
    assert (wide[:, 240:] == 7.0).all(), "lse written past total_q"


def test_mla_prefill_causal_and_context_chunks_merge(cuda):
    """MLA prefill as mla_attention_impl.py:347-398 runs it through FlashAttnVarlen: query
    / key head 192, value head 128, 16 heads (MHA).  The new tokens attend causally; each
    cached-context chunk is attended non-causally with its LSE; merge_attn_states of
    the two (out, lse) pairs equals the attention over the context and the new tokens
    together (end-aligned causal over all keys)."""
    from fastkernels_amd.candidate.L1.flash_attn_varlen import FlashAttnVarlen

    _flush("MLA prefill 192/128")
    h, d, dv = 16, 192, 128
    new_lens, ctx_lens = [300, 17, 1], [1000, 64, 0]
    g = torch.Generator().manual_seed(11)
    q = torch.randn(sum(new_lens), h, d, generator=g).to(torch.bfloat16).to(cuda)
    k_new = torch.randn(sum(new_lens), h, d, generator=g).to(torch.bfloat16).to(cuda)
    v_new = torch.randn(sum(new_lens), h, dv, generator=g).to(torch.bfloat16).to(cuda)
    k_ctx = torch.randn(sum(ctx_lens), h, d, generator=g).to(torch.bfloat16).to(cuda)
    v_ctx = torch.randn(sum(ctx_lens), h, dv, generator=g).to(torch.bfloat16).to(cuda)
    cu_q = torch.tensor([0] + list(np.cumsum(new_lens)), dtype=torch.int32, device=cuda)
    cu_c = torch.tensor([0] + list(np.cumsum(ctx_lens)), dtype=torch.int32, device=cuda)
    scale = d ** -0.5
    m = FlashAttnVarlen()
    suffix, suffix_lse = m(q, k_new, v_new, cu_q, cu_q, max(new_lens), max(new_lens), scale,
                           causal=True, return_softmax_lse=True)
    prefix, prefix_lse = m(q, k_ctx, v_ctx, cu_q, cu_c, max(new_lens), max(ctx_lens), scale,
                           causal=False, return_softmax_lse=True)
    torch.cuda.synchronize()
    f = lambda t: t.float().cpu().numpy()  # noqa: E731
    ref_s, ref_sl = oracle.varlen_prefill(f(q), f(k_new), f(v_new), f(cu_q).astype(np.int32),
                                          f(cu_q).astype(np.int32), scale, True, return_lse=True)
    ref_p, ref_pl = oracle.varlen_prefill(f(q), f(k_ctx), f(v_ctx), f(cu_q).astype(np.int32),
                                          f(cu_c).astype(np.int32), scale, False,
                                          return_lse=True)
    assert suffix.shape == (sum(new_lens), h, dv)
    _close(suffix, ref_s, 1e-2, "MLA causal")
    _close(prefix, ref_p, 1e-2, "MLA context chunk")
    _lse_close(suffix_lse, ref_sl, "MLA causal lse")
    _lse_close(prefix_lse, ref_pl, "MLA context lse")  # the empty context: -inf rows
    # merge (mla_attention_impl.py: merge_attn_states(prefix = context, suffix = new))
    merged = torch.empty_like(suffix)
    ops.merge_attn_states(merged, prefix, prefix_lse, suffix, suffix_lse, None)
    torch.cuda.synchronize()
    # the whole: per sequence, keys = context then new tokens, end-aligned causal
    ks, vs, cuk = [], [], [0]
    for i in range(len(new_lens)):
        c0, c1 = int(cu_c[i]), int(cu_c[i + 1])
        n0, n1 = int(cu_q[i]), int(cu_q[i + 1])
        ks += [f(k_ctx[c0:c1]), f(k_new[n0:n1])]
        vs += [f(v_ctx[c0:c1]), f(v_new[n0:n1])]
        cuk.append(cuk[-1] + (c1 - c0) + (n1 - n0))
    whole = oracle.varlen_prefill(f(q), np.concatenate(ks), np.concatenate(vs),
                                  f(cu_q).astype(np.int32), np.array(cuk, np.int32), scale, True)
    _close(merged, whole, 1e-2, "MLA merged = whole")


@pytest.mark.parametrize("d", [32, 72, 80, 96])
def test_varlen_prefill_padded_head_sizes(cuda, d):
    """Head sizes that are not multiples of 32 (72, 80: Qwen3-VL's and Qwen2.5-VL's vision
    encoders) or small (32, 96): dense keys, bidirectional (the vision encoder's form,
    MHA) and causal GQA, key split and single pass, with the LSE."""
    _flush(f"varlen prefill head {d}")
    for causal, hq, hk in ((False, 16, 16), (True, 16, 4)):
        q_lens, k_lens = ([1024, 300, 1], [1024, 300, 1]) if not causal else ([200, 9], [500, 9])
        q, k, v, cu_q, cu_k = _dense(cuda, q_lens, k_lens, hq, hk, d, seed=d)
        ref, ref_lse = _oracle_dense(q, k, v, cu_q, cu_k, d ** -0.5, causal, lse=True)
        for max_q in (max(q_lens), 20000):
            out, lse = _run_dense(q, k, v, cu_q, cu_k, max_q, d ** -0.5, causal, lse=True,
                                  max_k=max(k_lens))
            _close(out, ref, 1e-2, f"d={d} causal={causal} max_q={max_q}")
            _lse_close(lse, ref_lse, f"d={d} lse causal={causal} max_q={max_q}")


@pytest.mark.parametrize("d", [32, 72, 80, 96])
def test_paged_prefill_padded_head_sizes(cuda, d):
    """The same head sizes over a paged cache (16-token pages; chunks over cached
    prefixes, a prompt, the key split and the single pass)."""
    _flush(f"paged prefill head {d}")
    g = torch.Generator().manual_seed(200 + d)
    q_lens, k_lens, hq, hk, bs = [100, 33, 1], [100, 700, 60], 16, 4, 16
    pages = [(n + bs - 1) // bs for n in k_lens]
    nb = sum(pages) + 2
    perm = torch.randperm(nb, generator=g)
    bt = torch.full((3, max(pages)), -1, dtype=torch.int32)
    off = 0
    for i, pcount in enumerate(pages):
        bt[i, :pcount] = perm[off:off + pcount].to(torch.int32)
        off += pcount
    q = torch.randn(sum(q_lens), hq, d, generator=g).to(torch.bfloat16).to(cuda)
    kc = torch.randn(nb, bs, hk, d, generator=g).to(torch.bfloat16).to(cuda)
    vc = torch.randn(nb, bs, hk, d, generator=g).to(torch.bfloat16).to(cuda)
    cu_q = torch.tensor([0] + list(np.cumsum(q_lens)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(np.cumsum(k_lens)), dtype=torch.int32)
    ref = oracle.paged_prefill(q.float().cpu().numpy(), kc.float().cpu().numpy(),
                               vc.float().cpu().numpy(), bt.numpy(), cu_q.numpy(), cu_k.numpy(),
                               d ** -0.5)
    for max_q in (max(q_lens), 20000):
        out = torch.full_like(q, float("nan"))
        ops.paged_prefill(out, q, kc, vc, bt.to(cuda), cu_q.to(cuda), cu_k.to(cuda), max_q,
                          d ** -0.5, max_seqlen_k=max(k_lens))
        torch.cuda.synchronize()
        _close(out, ref, 1e-2, f"paged d={d} max_q={max_q}")


def test_flash_attn_prefill_candidate_vision_head_80(cuda):
    """FlashAttnPrefill(16, 16, 80), Qwen2.5-VL's vision attention (VisionAttention builds
    it at projection_size // num_heads = 1280 // 16, vision_attention.py:32,39): dense,
    non-causal over two images' patches (cu_seqlens), flat [N, heads * 80] inputs."""
    from fastkernels_amd.candidate.L1.flash_attn_prefill import FlashAttnPrefill

    _flush("FlashAttnPrefill vision head 80")
    lens = [1024, 576]
    q, k, v, cu, _ = _dense(cuda, lens, lens, 16, 16, 80, seed=80)
    mod = FlashAttnPrefill(16, 16, 80)
    out = mod(q.view(-1, 16 * 80), k.view(-1, 16 * 80), v.view(-1, 16 * 80), cu, cu, max(lens),
              max(lens), causal=False)
    torch.cuda.synchronize()
    ref = _oracle_dense(q, k, v, cu, cu, 80 ** -0.5, False)
    _close(out.view(-1, 16, 80), ref, 1e-2, "vision head 80")
