"""Writes the small golden fixtures of the decode-step ops (tests/golden/*.npz).

Inputs are drawn from numpy's PCG64 with fixed seeds and rounded to the op's
dtype; expected outputs come from the CPU oracle (oracle/), which
tests/test_oracle.py pins against library routines, closed forms and
invariants.  The fixtures freeze those outputs so that later changes to the
oracle or the kernels are checked against the same vectors.  Regenerate with
``python tests/golden/make_golden.py`` (only when the oracle is intentionally
changed; tests/test_golden.py fails if a regeneration would differ).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

import oracle  # noqa: E402


def bf16(x):
    return oracle.round_to(np.asarray(x, np.float32), "bf16")


def cases() -> dict[str, dict[str, np.ndarray]]:
    out = {}
    r = np.random.default_rng(1001)
    # fused add + RMSNorm and plain RMSNorm, bf16, hidden 256 (vector path) and 200 (scalar path)
    for h in (256, 200):
        x, res = bf16(r.standard_normal((6, h))), bf16(r.standard_normal((6, h)))
        w = bf16(1 + 0.1 * r.standard_normal(h))
        o, nr = oracle.rms_norm(x, w, 1e-6, "bf16", residual=res)
        out[f"rmsnorm_h{h}"] = dict(x=x, residual=res, weight=w, eps=np.float32(1e-6),
                                    out_fused=o, new_residual=nr,
                                    out_plain=oracle.rms_norm(x, w, 1e-6, "bf16"))
    # rotary, NeoX and GPT-J, bf16 q [5, 4*64], k [5, 2*64], theta 1e4, fp32 cache
    cs = oracle.rope_cos_sin_cache(64, 160, 1e4)
    pos = np.array([0, 1, 7, 150, 159], np.int64)
    q, k = bf16(r.standard_normal((5, 256))), bf16(r.standard_normal((5, 128)))
    for neox in (True, False):
        oq, ok = oracle.rotary(pos, q, k, 64, cs, neox, "bf16")
        out[f"rotary_{'neox' if neox else 'gptj'}"] = dict(positions=pos, q=q, k=k, cos_sin=cs,
                                                           out_q=oq, out_k=ok)
    # store_kvcache: bf16 bit patterns, 12 tokens into 4 blocks x 8 slots, -1 skips
    key = r.integers(-32768, 32767, (12, 2, 16)).astype(np.int16)
    val = r.integers(-32768, 32767, (12, 2, 16)).astype(np.int16)
    slots = r.permutation(32)[:12].astype(np.int64)
    slots[[2, 9]] = -1
    kc = np.zeros((4, 8, 2, 16), np.int16)
    ek, ev = oracle.store_kvcache(key, val, kc, kc, slots)
    out["store_kvcache"] = dict(key=key, value=val, slot_mapping=slots, k_cache=ek, v_cache=ev)
    # paged decode bf16: 5 seqs (one empty), Hq 8, Hk 2, D 128, block 16, pool 20
    lens = np.array([33, 0, 1, 70, 16], np.int32)
    nb, bs = 11, 16
    q = bf16(r.standard_normal((5, 8, 128)))
    kcache = bf16(r.standard_normal((nb, bs, 2, 128)))
    vcache = bf16(r.standard_normal((nb, bs, 2, 128)))
    perm = r.permutation(nb)
    bt = -np.ones((5, 5), np.int32)
    off = 0
    for i, n in enumerate(lens):
        p = (n + bs - 1) // bs
        bt[i, :p] = perm[off:off + p]
        off += p
    scale = np.float32(1 / np.sqrt(128))
    out["paged_decode_bf16"] = dict(q=q, k_cache=kcache, v_cache=vcache, block_tables=bt,
                                    ctx_lens=lens, scale=scale,
                                    out=oracle.paged_decode(q, kcache, vcache, bt, lens,
                                                            float(scale)).astype(np.float32))
    # paged decode fp8 e4m3fn KV with per-kv-head scales, Hq 16, Hk 2
    ks = np.array([0.03, 0.07], np.float32)
    vs = np.array([0.05, 0.02], np.float32)
    q8 = bf16(r.standard_normal((5, 16, 128)))
    k8 = oracle.fp8_e4m3fn_encode(r.standard_normal((nb, bs, 2, 128)) / ks.reshape(1, 1, 2, 1))
    v8 = oracle.fp8_e4m3fn_encode(r.standard_normal((nb, bs, 2, 128)) / vs.reshape(1, 1, 2, 1))
    out["paged_decode_fp8"] = dict(q=q8, k_cache=k8, v_cache=v8, block_tables=bt, ctx_lens=lens,
                                   scale=scale, k_scale=ks, v_scale=vs,
                                   out=oracle.paged_decode(q8, k8, v8, bt, lens, float(scale), ks,
                                                           vs).astype(np.float32))
    # SiLU-and-mul bf16 [6, 2*96] and a scalar-path width [3, 2*13]
    for d in (96, 13):
        x = bf16(3 * r.standard_normal((6, 2 * d)))
        out[f"silu_and_mul_d{d}"] = dict(x=x, out=oracle.silu_and_mul(x, "bf16"))
    # (Fixtures below were added after the ones above; their draws come from
    # their own generator so the earlier fixtures keep their values.)
    r2 = np.random.default_rng(2002)
    # merge_attn_states bf16 [T 6, H 3, D 64] with lse specials; suffix-only tail at 5
    po, so = bf16(r2.standard_normal((6, 3, 64))), bf16(r2.standard_normal((6, 3, 64)))
    pl = (3 * r2.standard_normal((3, 6))).astype(np.float32)
    sl = (3 * r2.standard_normal((3, 6))).astype(np.float32)
    pl[0, 0] = -np.inf
    sl[1, 1] = -np.inf
    pl[2, 2] = sl[2, 2] = -np.inf
    pl[1, 3] = np.inf
    mo, ml = oracle.merge_attn_states(po, pl, so, sl, "bf16", prefill_tokens_with_context=5)
    out["merge_attn_states"] = dict(prefix=po, prefix_lse=pl, suffix=so, suffix_lse=sl,
                                    prefill_tokens=np.int64(5), out=mo, out_lse=ml)
    # paged prefill bf16: chunks (q_len, k_len) = (5, 5), (1, 17), (9, 30), (4, 2); Hq 8, Hk 2
    q_lens, k_lens = [5, 1, 9, 4], [5, 17, 30, 2]
    bs = 16
    pages = [(k + bs - 1) // bs for k in k_lens]
    nbp = sum(pages) + 1
    permp = r2.permutation(nbp)
    btp = -np.ones((4, max(pages)), np.int32)
    off = 0
    for i, p in enumerate(pages):
        btp[i, :p] = permp[off:off + p]
        off += p
    cu_q = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(k_lens)]).astype(np.int32)
    qp = bf16(r2.standard_normal((int(cu_q[-1]), 8, 128)))
    kcp = bf16(r2.standard_normal((nbp, bs, 2, 128)))
    vcp = bf16(r2.standard_normal((nbp, bs, 2, 128)))
    out["paged_prefill_bf16"] = dict(
        q=qp, k_cache=kcp, v_cache=vcp, block_tables=btp, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k,
        scale=scale, out=oracle.paged_prefill(qp, kcp, vcp, btp, cu_q, cu_k,
                                              float(scale)).astype(np.float32))
    # per-head q/k RMSNorm + NeoX rotary (the fused attention prologue), bf16, D 64
    cs64 = oracle.rope_cos_sin_cache(64, 64, 1e4)
    posq = np.array([0, 3, 63, 17], np.int64)
    qh, kh = bf16(r2.standard_normal((4, 4 * 64))), bf16(r2.standard_normal((4, 2 * 64)))
    qw, kw = bf16(1 + 0.2 * r2.standard_normal(64)), bf16(1 + 0.2 * r2.standard_normal(64))
    qn = oracle.rms_norm(qh.reshape(4, 4, 64), qw, 1e-6, "bf16").reshape(4, -1)
    kn = oracle.rms_norm(kh.reshape(4, 2, 64), kw, 1e-6, "bf16").reshape(4, -1)
    oq, ok = oracle.rotary(posq, qn, kn, 64, cs64, True, "bf16")
    out["qk_norm_rope"] = dict(positions=posq, q=qh, k=kh, q_weight=qw, k_weight=kw,
                               cos_sin=cs64, eps=np.float32(1e-6), out_q=oq, out_k=ok)
    # Sliding window + attention sinks (flash-attn window_size = (w, 0), s_aux) on the
    # inputs of paged_decode_bf16 (window 20) and paged_prefill_bf16 (window 6): these
    # fixtures hold only the window, the sinks (their own generator) and the output.
    r3 = np.random.default_rng(2003)
    sinks8 = (2 * r3.standard_normal(8)).astype(np.float32)
    out["paged_decode_window_sinks"] = dict(
        window_left=np.int64(20), sinks=sinks8,
        out=oracle.paged_decode(q, kcache, vcache, bt, lens, float(scale), window_left=20,
                                sinks=sinks8).astype(np.float32))
    out["paged_prefill_window_sinks"] = dict(
        window_left=np.int64(6), sinks=sinks8,
        out=oracle.paged_prefill(qp, kcp, vcp, btp, cu_q, cu_k, float(scale), window_left=6,
                                 sinks=sinks8).astype(np.float32))
    return out


def main():
    for name, arrays in cases().items():
        np.savez_compressed(HERE / f"{name}.npz", **arrays)
        print(name, sum(a.nbytes for a in arrays.values()), "bytes")


if __name__ == "__main__":
    main()
