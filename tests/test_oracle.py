"""Pins the CPU oracle (``oracle/``) before it is trusted as the checker.

The reference holds no golden vectors for this path (its tests pin harness
behaviour only), so each oracle function is pinned by checks independent of
its own formula:
  number formats   exhaustive / randomized agreement with torch's bf16, fp16 and
                   float8_e4m3fn conversions (library routines);
  rms_norm         torch.nn.functional.rms_norm (library), a closed-form scale
                   invariance, the bit-exact residual rule, eps-dominated rows;
  rotary           hand-computed known-answer vectors for both pairings, the
                   cos/sin cache against float64 math, norm preservation, the
                   relative-position property, position 0 = identity;
  store_kvcache    a brute-force per-slot loop and the untouched-slot invariant;
  paged decode     torch scaled_dot_product_attention in float64 (library) with
                   repeat_interleave GQA, closed forms (uniform scores -> mean of V,
                   one dominant key -> its V row, empty -> 0), page-permutation
                   invariance, split-context merge == unsplit;
  silu_and_mul     torch.nn.functional.silu (library) with the reference's
                   rounding points;
  paged_prefill    torch SDPA (float64) with is_causal when the chunk is the whole
                   context and with an explicit bottom-right mask otherwise;
                   q_len = 1 equals paged_decode; a query's output does not depend
                   on keys after its position; a planted top-left mask is caught;
  varlen_prefill   torch SDPA (float64) per sequence over its dense K/V slice with the
                   end-aligned mask (and without it, non-causal); equal to
                   paged_prefill on the same keys scattered into shuffled pages; a
                   planted cu_seqlens_q / cu_seqlens_k swap is caught;
  torch_path       decode_torch (the CPU baseline leg) against paged_decode;
  merge_attn_states  attention over a key set split in two and merged equals
                   torch SDPA over the whole set, and out_lse equals
                   torch.logsumexp of all scores (library); the special cases
                   (one side empty, both empty, +inf lse, suffix-only tokens).
Planted-mistake tests show the checks reject plausible slips (wrong GQA head
mapping, dropped eps, swapped rotary pairing, a wrong sign).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle

RNG = np.random.default_rng(1234)


# ---------------------------------------------------------------------------
# Number formats
# ---------------------------------------------------------------------------
def test_bf16_decode_exhaustive():
    bits = np.arange(65536, dtype=np.uint16)
    ours = oracle.bf16_bits_to_f32(bits)
    theirs = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).float().numpy()
    same = (ours.view(np.uint32) == theirs.view(np.uint32)) | (np.isnan(ours) & np.isnan(theirs))
    assert same.all()


def test_bf16_round_matches_torch():
    x = np.concatenate([
        RNG.standard_normal(200_000).astype(np.float32) * 10.0 ** RNG.integers(-30, 30, 200_000),
        np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40, 3.4e38, 1.0 + 2 ** -8,
                  1.0 + 3 * 2 ** -8, 1.0 + 2 ** -9], np.float32),
        # exact ties at several exponents
        (np.arange(1, 2000, dtype=np.float32) * 2.0 ** -8 + 1.0).astype(np.float32),
    ]).astype(np.float32)
    ours = oracle.f32_to_bf16_bits(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    assert oracle.f32_to_bf16_bits(np.array([np.nan], np.float32))[0] == 0x7FC0


def test_f16_round_matches_torch():
    x = (RNG.standard_normal(100_000) * 100).astype(np.float32)
    theirs = torch.from_numpy(x).half().float().numpy()
    assert np.array_equal(oracle.round_to(x, "f16"), theirs)


def test_e4m3fn_table_matches_torch_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    theirs = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    ours = oracle.fp8_e4m3fn_decode(codes)
    assert np.array_equal(np.isnan(ours), np.isnan(theirs))
    ok = ~np.isnan(ours)
    assert np.array_equal(ours[ok], theirs[ok])
    assert np.nanmax(ours) == 448.0 and np.isnan(ours[0x7F]) and np.isnan(ours[0xFF])
    assert ours[0x01] == 2.0 ** -9 and ours[0x08] == 2.0 ** -6  # smallest subnormal / normal


def test_e4m3fn_encode_matches_torch():
    x = np.concatenate([RNG.standard_normal(100_000) * 30, RNG.standard_normal(1000) * 1e-3,
                        [0.0, 447.0, 448.0, 464.0, 1e6, -1e6, 2.0 ** -10, 2.0 ** -9 * 1.5]])
    xc = np.clip(x, -448, 448).astype(np.float32)
    theirs = torch.from_numpy(xc).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    ours = oracle.fp8_e4m3fn_encode(x)
    assert np.array_equal(ours, theirs)
    # saturation (Triton's satfinite store) and NaN with its sign
    assert list(oracle.fp8_e4m3fn_encode(np.array([np.inf, -np.inf, 1e9, np.nan, -np.nan]))) == \
        [0x7E, 0xFE, 0x7E, 0x7F, 0xFF]


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------
def _norm_inputs(t=16, h=256, scale=1.0):
    x = (RNG.standard_normal((t, h)) * scale).astype(np.float32)
    r = (RNG.standard_normal((t, h)) * scale).astype(np.float32)
    w = (1 + 0.1 * RNG.standard_normal(h)).astype(np.float32)
    return x, r, w


def test_rms_norm_f32_matches_torch_rms_norm():
    x, r, w = _norm_inputs()
    ours = oracle.rms_norm(x, w, 1e-6, "f32")
    theirs = F.rms_norm(torch.from_numpy(x), (x.shape[-1],), torch.from_numpy(w), eps=1e-6)
    np.testing.assert_allclose(ours, theirs.numpy(), rtol=2e-6, atol=2e-6)
    # Fused form: the norm of the fp32 sum.
    ours_f, res = oracle.rms_norm(x, w, 1e-6, "f32", residual=r)
    theirs_f = F.rms_norm(torch.from_numpy(x + r), (x.shape[-1],), torch.from_numpy(w), eps=1e-6)
    np.testing.assert_allclose(ours_f, theirs_f.numpy(), rtol=2e-6, atol=2e-6)
    assert np.array_equal(res, x + r)


def test_rms_norm_eps_dominated_rows():
    """Tiny rows where eps dominates the variance: catches a dropped or misplaced eps."""
    x, _, w = _norm_inputs(scale=1e-4)
    ours = oracle.rms_norm(x, w, 1e-6, "f32")
    theirs = F.rms_norm(torch.from_numpy(x), (x.shape[-1],), torch.from_numpy(w), eps=1e-6).numpy()
    np.testing.assert_allclose(ours, theirs, rtol=1e-5, atol=1e-9)
    no_eps = oracle.rms_norm(x, w, 0.0, "f32")
    assert not np.allclose(no_eps, theirs, rtol=1e-3), "planted mistake (eps dropped) not caught"


def test_rms_norm_bf16_residual_and_scale_invariance():
    x, r, w = _norm_inputs()
    xb, rb, wb = (oracle.round_to(a, "bf16") for a in (x, r, w))
    out, res = oracle.rms_norm(xb, wb, 1e-6, "bf16", residual=rb)
    # new residual == bf16(x + r): torch's bf16 add (fp32 sum, one rounding).
    t = (torch.from_numpy(xb).bfloat16() + torch.from_numpy(rb).bfloat16()).float().numpy()
    assert np.array_equal(res, t)
    # Closed form: with eps = 0, scaling x by 4 (exact in fp32, sqrt(16 v) = 4 sqrt(v))
    # leaves the output bit-identical.
    a = oracle.rms_norm(xb, wb, 0.0, "bf16")
    b = oracle.rms_norm(xb * 4, wb, 0.0, "bf16")
    assert np.array_equal(a, b)
    # Output matches torch's forward_native op sequence in bf16 to one bf16 ulp.
    xt = torch.from_numpy(xb).bfloat16().float()
    ref = (xt * torch.rsqrt(xt.pow(2).mean(-1, keepdim=True) + 1e-6)).bfloat16() * \
        torch.from_numpy(wb).bfloat16()
    np.testing.assert_allclose(oracle.rms_norm(xb, wb, 1e-6, "bf16"), ref.float().numpy(),
                               rtol=8e-3, atol=1e-6)


# ---------------------------------------------------------------------------
# Rotary
# ---------------------------------------------------------------------------
def test_rotary_known_answers():
    """head_dim 4, theta 10000: inv_freq = [1, 0.01].  x = e0 at position 1:
    NeoX pairs (0,2),(1,3) -> [cos 1, 0, sin 1, 0]; GPT-J pairs (0,1),(2,3) -> [cos 1, sin 1, 0, 0]."""
    cs = oracle.rope_cos_sin_cache(4, 2, 10000.0)
    np.testing.assert_allclose(cs[1], [math.cos(1), math.cos(0.01), math.sin(1), math.sin(0.01)],
                               rtol=1e-6)
    x = np.array([[1.0, 0.0, 0.0, 0.0]], np.float32)
    neox, _ = oracle.rotary(np.array([1]), x, None, 4, cs, True, "f32")
    gptj, _ = oracle.rotary(np.array([1]), x, None, 4, cs, False, "f32")
    np.testing.assert_allclose(neox[0], [math.cos(1), 0, math.sin(1), 0], atol=1e-6)
    np.testing.assert_allclose(gptj[0], [math.cos(1), math.sin(1), 0, 0], atol=1e-6)
    y = np.array([[0.0, 0.0, 1.0, 0.0]], np.float32)  # second half: -sin lands in slot 0
    neox_y, _ = oracle.rotary(np.array([1]), y, None, 4, cs, True, "f32")
    np.testing.assert_allclose(neox_y[0], [-math.sin(1), 0, math.cos(1), 0], atol=1e-6)


def test_rotary_cache_vs_float64_math():
    d, theta = 128, 1e6
    cs = oracle.rope_cos_sin_cache(d, 4097, theta)
    inv = 1.0 / theta ** (np.arange(0, d, 2) / d)
    ang = np.outer(np.arange(4097), inv)
    # float32 angles: error grows with |angle| ~ position * 1e-7 relative.
    np.testing.assert_allclose(cs[:, :d // 2], np.cos(ang), atol=2e-3)
    np.testing.assert_allclose(cs[:, d // 2:], np.sin(ang), atol=2e-3)
    np.testing.assert_allclose(cs[:64, :d // 2], np.cos(ang[:64]), atol=1e-5)


@pytest.mark.parametrize("neox", [True, False])
def test_rotary_invariants(neox):
    d, t = 64, 32
    cs = oracle.rope_cos_sin_cache(d, 512, 10000.0)
    q = RNG.standard_normal((t, 2 * d)).astype(np.float32)
    k = RNG.standard_normal((t, d)).astype(np.float32)
    pos = RNG.integers(0, 400, t)
    rq, rk = oracle.rotary(pos, q, k, d, cs, neox, "f32")
    # norm preservation per head
    np.testing.assert_allclose(np.linalg.norm(rq.reshape(t, 2, d), axis=-1),
                               np.linalg.norm(q.reshape(t, 2, d), axis=-1), rtol=1e-5)
    # position 0 is the identity
    r0, _ = oracle.rotary(np.zeros(t, np.int64), q, None, d, cs, neox, "f32")
    assert np.array_equal(r0, q)
    # relative position: <rot(q, p), rot(k, p')> depends on p - p' only
    qa, ka = oracle.rotary(pos, q[:, :d], k, d, cs, neox, "f32")
    qb, kb = oracle.rotary(pos + 50, q[:, :d], k, d, cs, neox, "f32")
    sa = np.einsum("td,sd->ts", qa, ka)
    sb = np.einsum("td,sd->ts", qb, kb)
    np.testing.assert_allclose(sa, sb, atol=2e-4)
    # planted mistake: "x*c + y*s" in the first output is not a rotation; the
    # norm-preservation check above rejects it.
    half = d // 2
    c_, s_ = cs[pos][:, None, :half], cs[pos][:, None, half:]
    x1, x2 = q.reshape(t, 2, d)[..., :half], q.reshape(t, 2, d)[..., half:]
    mutant = np.concatenate([x1 * c_ + x2 * s_, x2 * c_ + x1 * s_], -1)
    assert not np.allclose(np.linalg.norm(mutant, axis=-1),
                           np.linalg.norm(q.reshape(t, 2, d), axis=-1), rtol=1e-3)


# ---------------------------------------------------------------------------
# store_kvcache
# ---------------------------------------------------------------------------
def test_store_kvcache_vs_loop():
    nb, bs, hk, d, n = 6, 8, 2, 4, 20
    key = RNG.integers(-30000, 30000, (n, hk, d)).astype(np.int16)
    val = RNG.integers(-30000, 30000, (n, hk, d)).astype(np.int16)
    kc = RNG.integers(-5, 5, (nb, bs, hk, d)).astype(np.int16)
    vc = kc.copy()
    slots = RNG.permutation(nb * bs)[:n]
    slots[[1, 7, 11]] = -1
    ek, ev = oracle.store_kvcache(key, val, kc, vc, slots)
    bk, bv = kc.copy(), vc.copy()
    for i, s in enumerate(slots):
        if s < 0:
            continue
        bk[s // bs, s % bs] = key[i]
        bv[s // bs, s % bs] = val[i]
    assert np.array_equal(ek, bk) and np.array_equal(ev, bv)
    untouched = np.setdiff1d(np.arange(nb * bs), slots[slots >= 0])
    assert np.array_equal(ek.reshape(nb * bs, -1)[untouched], kc.reshape(nb * bs, -1)[untouched])


def test_store_kvcache_hnd_is_the_nhd_store_transposed():
    """The HND store equals the NHD store with the cache's head and slot axes swapped
    (a closed-form relation between the two layouts); a swapped (page, head) index is
    caught."""
    nb, bs, hk, d, n = 5, 8, 3, 4, 25
    key = RNG.integers(-30000, 30000, (n, hk, d)).astype(np.int16)
    val = RNG.integers(-30000, 30000, (n, hk, d)).astype(np.int16)
    slots = RNG.permutation(nb * bs)[:n]
    slots[[0, 9]] = -1
    slots[4] = nb * bs + 3  # past the cache: skipped
    kc_hnd = RNG.integers(-5, 5, (nb, hk, bs, d)).astype(np.int16)
    vc_hnd = kc_hnd.copy()
    ek, ev = oracle.store_kvcache_hnd(key, val, kc_hnd, vc_hnd, slots, bs)
    nhd_k = np.ascontiguousarray(kc_hnd.transpose(0, 2, 1, 3))
    nhd_v = np.ascontiguousarray(vc_hnd.transpose(0, 2, 1, 3))
    sl = np.where(slots >= nb * bs, -1, slots)
    rk, rv = oracle.store_kvcache(key, val, nhd_k, nhd_v, sl)
    assert np.array_equal(ek, rk.transpose(0, 2, 1, 3))
    assert np.array_equal(ev, rv.transpose(0, 2, 1, 3))
    wrong = kc_hnd.copy()
    for i, s_ in enumerate(sl):
        if s_ >= 0:
            wrong[s_ // bs, :, s_ % bs] = key[i][::-1]  # heads reversed
    assert not np.array_equal(wrong, ek)


# ---------------------------------------------------------------------------
# Paged decode attention
# ---------------------------------------------------------------------------
def _decode_case(b=4, hq=8, hk=2, d=16, bs=4, nb=64, seed=0, lens=None):
    r = np.random.default_rng(seed)
    lens = np.array(lens if lens is not None else r.integers(1, 40, b))
    b = len(lens)
    q = r.standard_normal((b, hq, d)).astype(np.float32)
    kc = r.standard_normal((nb, bs, hk, d)).astype(np.float32)
    vc = r.standard_normal((nb, bs, hk, d)).astype(np.float32)
    perm = r.permutation(nb)
    width = int(max(1, max((n + bs - 1) // bs for n in lens)))
    bt = -np.ones((b, width), np.int32)
    off = 0
    for i, n in enumerate(lens):
        p = (n + bs - 1) // bs
        bt[i, :p] = perm[off:off + p]
        off += p
    return q, kc, vc, bt, lens.astype(np.int32)


def _sdpa_ref(q, kc, vc, bt, lens, scale, head_of):
    out = np.zeros(q.shape, np.float64)
    for i in range(q.shape[0]):
        n = int(lens[i])
        ks = torch.from_numpy(oracle.gather_seq(kc, bt[i], n)).double()
        vs = torch.from_numpy(oracle.gather_seq(vc, bt[i], n)).double()
        hq = q.shape[1]
        idx = torch.tensor([head_of(h) for h in range(hq)])
        kh = ks[:, idx].transpose(0, 1).contiguous()  # [Hq, n, D]
        vh = vs[:, idx].transpose(0, 1).contiguous()
        qh = torch.from_numpy(q[i]).double()[:, None, :]
        out[i] = F.scaled_dot_product_attention(qh, kh, vh, scale=scale)[:, 0].numpy()
    return out


def test_paged_decode_vs_torch_sdpa():
    q, kc, vc, bt, lens = _decode_case()
    scale = 1 / math.sqrt(16)
    grp = q.shape[1] // kc.shape[2]
    ours = oracle.paged_decode(q, kc, vc, bt, lens, scale)
    ref = _sdpa_ref(q, kc, vc, bt, lens, scale, lambda h: h // grp)  # repeat_interleave
    np.testing.assert_allclose(ours, ref, rtol=1e-10, atol=1e-12)
    # planted mistake: GQA head h -> kv head h % Hk is caught by the same check
    wrong = _sdpa_ref(q, kc, vc, bt, lens, scale, lambda h: h % kc.shape[2])
    assert not np.allclose(ours, wrong, atol=1e-3), "planted mistake (GQA mapping) not caught"


def test_paged_decode_closed_forms():
    q, kc, vc, bt, lens = _decode_case(lens=[0, 5, 13])
    out = oracle.paged_decode(q, kc, vc, bt, lens, 0.25)
    assert np.array_equal(out[0], np.zeros_like(out[0]))  # empty context -> 0
    # uniform scores (q = 0) -> the mean of the visible V rows
    q0 = np.zeros_like(q)
    out0 = oracle.paged_decode(q0, kc, vc, bt, lens, 0.25)
    for i in (1, 2):
        vs = oracle.gather_seq(vc, bt[i], int(lens[i])).astype(np.float64)
        np.testing.assert_allclose(out0[i], np.repeat(vs.mean(0), 4, axis=0), atol=1e-12)
    # one dominant key -> its V row: q of every head points at token 3's key of its kv head
    i, tgt, bs, grp = 2, 3, kc.shape[1], q.shape[1] // kc.shape[2]
    page, slot = bt[i, tgt // bs], tgt % bs
    qd = q.copy()
    for h in range(q.shape[1]):
        kt = kc[page, slot, h // grp].astype(np.float64)
        qd[i, h] = 200.0 * kt / (kt @ kt)
    outd = oracle.paged_decode(qd, kc, vc, bt, lens, 1.0)
    np.testing.assert_allclose(outd[i], np.repeat(vc[page, slot], grp, axis=0), atol=1e-6)


def test_paged_decode_page_permutation_invariance():
    q, kc, vc, bt, lens = _decode_case(seed=3)
    base = oracle.paged_decode(q, kc, vc, bt, lens, 0.3)
    perm = np.random.default_rng(9).permutation(kc.shape[0])  # page p moves to perm[p]
    kc2, vc2 = np.empty_like(kc), np.empty_like(vc)
    kc2[perm], vc2[perm] = kc, vc
    bt2 = np.where(bt >= 0, perm[np.maximum(bt, 0)], -1).astype(np.int32)
    np.testing.assert_allclose(oracle.paged_decode(q, kc2, vc2, bt2, lens, 0.3), base, atol=0)


def _sdpa_sink_window_ref(q, kc, vc, bt, lens, scale, sinks=None, window_left=-1):
    """Brute force for sinks and windows in float64 torch: the window slices each
    sequence's keys to its last window_left + 1; a sink is one more key per query
    head whose score is exactly the sink logit (k = sink / (scale |q|^2) q) and whose
    value row is zero, so it joins the denominator only."""
    out = np.zeros(q.shape, np.float64)
    hq, hk = q.shape[1], kc.shape[2]
    idx = torch.tensor([h // (hq // hk) for h in range(hq)])
    for i in range(q.shape[0]):
        n = int(lens[i])
        lo = max(0, n - 1 - window_left) if window_left >= 0 else 0
        ks = torch.from_numpy(oracle.gather_seq(kc, bt[i], n)[lo:]).double()
        vs = torch.from_numpy(oracle.gather_seq(vc, bt[i], n)[lo:]).double()
        kh = ks[:, idx].transpose(0, 1).contiguous()  # [Hq, n', D]
        vh = vs[:, idx].transpose(0, 1).contiguous()
        qh = torch.from_numpy(q[i]).double()[:, None, :]  # [Hq, 1, D]
        if sinks is not None:
            qq = torch.from_numpy(q[i]).double()
            ke = (torch.from_numpy(np.asarray(sinks, np.float64))[:, None] * qq
                  / (scale * (qq * qq).sum(-1, keepdim=True)))
            kh = torch.cat([kh, ke[:, None, :]], 1)
            vh = torch.cat([vh, torch.zeros(hq, 1, vh.shape[2], dtype=vh.dtype)], 1)
        if kh.shape[1] == 0:
            continue
        out[i] = F.scaled_dot_product_attention(qh, kh, vh, scale=scale)[:, 0].numpy()
    return out


def test_paged_decode_sinks_vs_torch():
    """Sinks: against SDPA with one zero-value key per head scoring the sink; -inf
    sinks change nothing; a dominant sink drives the row to 0; an empty row stays 0."""
    q, kc, vc, bt, lens = _decode_case(seed=5, lens=[0, 1, 13, 37])
    sinks = np.array([0.5, -1.0, 2.0, 0.0, 1.5, -3.0, 4.0, 0.25])[:q.shape[1]]
    ours = oracle.paged_decode(q, kc, vc, bt, lens, 0.3, sinks=sinks)
    ref = _sdpa_sink_window_ref(q, kc, vc, bt, lens, 0.3, sinks=sinks)
    np.testing.assert_allclose(ours, ref, rtol=1e-9, atol=1e-12)
    assert np.array_equal(ours[0], np.zeros_like(ours[0]))
    none = oracle.paged_decode(q, kc, vc, bt, lens, 0.3)
    np.testing.assert_allclose(
        oracle.paged_decode(q, kc, vc, bt, lens, 0.3, sinks=np.full(q.shape[1], -np.inf)), none,
        rtol=0, atol=0)
    big = oracle.paged_decode(q, kc, vc, bt, lens, 0.3, sinks=np.full(q.shape[1], 200.0))
    assert np.abs(big).max() < 1e-40
    # a dropped sink is caught (the sinks move the rows)
    assert not np.allclose(ours[2], none[2], atol=1e-3)


@pytest.mark.parametrize("window_left", [0, 1, 5, 12, 36, 100])
def test_paged_decode_window_vs_torch(window_left):
    """Sliding window: the last window_left + 1 keys, against SDPA on the sliced
    sequence (window 0 is the last V row; a window past the start is no window),
    with and without sinks; a window one key short is caught."""
    q, kc, vc, bt, lens = _decode_case(seed=6, lens=[1, 13, 37])
    ours = oracle.paged_decode(q, kc, vc, bt, lens, 0.3, window_left=window_left)
    ref = _sdpa_sink_window_ref(q, kc, vc, bt, lens, 0.3, window_left=window_left)
    np.testing.assert_allclose(ours, ref, rtol=1e-9, atol=1e-12)
    sinks = np.linspace(-1, 2, q.shape[1])
    np.testing.assert_allclose(
        oracle.paged_decode(q, kc, vc, bt, lens, 0.3, window_left=window_left, sinks=sinks),
        _sdpa_sink_window_ref(q, kc, vc, bt, lens, 0.3, sinks=sinks, window_left=window_left),
        rtol=1e-9, atol=1e-12)
    grp = q.shape[1] // kc.shape[2]
    for i, n in enumerate(lens):
        if window_left == 0:
            last = oracle.gather_seq(vc, bt[i], int(n))[-1].astype(np.float64)
            np.testing.assert_allclose(ours[i], np.repeat(last, grp, axis=0), atol=1e-12)
        if window_left >= n - 1:
            np.testing.assert_allclose(ours[i], oracle.paged_decode(q, kc, vc, bt, lens, 0.3)[i],
                                       atol=0, rtol=0)
    if 1 <= window_left < 36:
        short = _sdpa_sink_window_ref(q, kc, vc, bt, lens, 0.3, window_left=window_left - 1)
        assert not np.allclose(ours[2], short[2], atol=1e-3), "off-by-one window not caught"


@pytest.mark.parametrize("part", [1, 3, 4, 16, 1000])
def test_split_merge_equals_unsplit(part):
    q, kc, vc, bt, lens = _decode_case(seed=4, lens=[37])
    k = oracle.gather_seq(kc, bt[0], 37)
    v = oracle.gather_seq(vc, bt[0], 37)
    whole = oracle.attend_one(q[0], k, v, 0.3)
    merged = oracle.merge_partials(oracle.attend_partials(q[0], k, v, 0.3, part))
    np.testing.assert_allclose(merged, whole, rtol=1e-12, atol=1e-13)


def test_fp8_dequant_matches_torch():
    codes = RNG.integers(0, 256, (3, 4, 2, 8)).astype(np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0  # no NaN codes
    scale = np.array([0.05, 0.02], np.float32)
    ours = oracle.dequant_kv(codes, scale, "bf16")
    t = torch.from_numpy(codes).view(torch.float8_e4m3fn).float() * torch.from_numpy(scale).view(1, 1, 2, 1)
    assert np.array_equal(ours, t.bfloat16().float().numpy())
    # One per-tensor scale (the reference's FP8_PER_TENSOR) applies to every kv head,
    # as a 0-d or a size-1 array.
    t1 = torch.from_numpy(codes).view(torch.float8_e4m3fn).float() * 0.05
    for s in (np.float32(0.05), np.array([0.05], np.float32)):
        assert np.array_equal(oracle.dequant_kv(codes, s, "bf16"), t1.bfloat16().float().numpy())
    with pytest.raises(ValueError):
        oracle.dequant_kv(codes, np.ones(3, np.float32), "bf16")


# ---------------------------------------------------------------------------
# paged prefill
# ---------------------------------------------------------------------------
def _prefill_case(seed=21, q_lens=(5, 1, 9), k_lens=(5, 17, 30), hq=4, hk=2, d=16, bs=8):
    rng = np.random.default_rng(seed)
    pages = [(k + bs - 1) // bs for k in k_lens]
    nb = sum(pages) + 2
    perm = rng.permutation(nb)
    bt = np.full((len(k_lens), max(pages)), -1, np.int32)
    off = 0
    for i, p in enumerate(pages):
        bt[i, :p] = perm[off:off + p]
        off += p
    kc = rng.standard_normal((nb, bs, hk, d)).astype(np.float32)
    vc = rng.standard_normal((nb, bs, hk, d)).astype(np.float32)
    cu_q = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(k_lens)]).astype(np.int32)
    q = rng.standard_normal((int(cu_q[-1]), hq, d)).astype(np.float32)
    return q, kc, vc, bt, cu_q, cu_k


def test_paged_prefill_vs_torch_sdpa():
    q, kc, vc, bt, cu_q, cu_k = _prefill_case()
    scale = 0.3
    ours = oracle.paged_prefill(q, kc, vc, bt, cu_q, cu_k, scale)
    hq, hk = q.shape[1], kc.shape[2]
    for i in range(len(cu_q) - 1):
        qs, qe = int(cu_q[i]), int(cu_q[i + 1])
        kl = int(cu_k[i + 1] - cu_k[i])
        ql = qe - qs
        k = torch.from_numpy(oracle.gather_seq(kc, bt[i], kl)).double()
        v = torch.from_numpy(oracle.gather_seq(vc, bt[i], kl)).double()
        k = k.repeat_interleave(hq // hk, dim=1).transpose(0, 1)   # [hq, kl, d]
        v = v.repeat_interleave(hq // hk, dim=1).transpose(0, 1)
        qq = torch.from_numpy(q[qs:qe]).double().transpose(0, 1)   # [hq, ql, d]
        if ql == kl:
            ref = F.scaled_dot_product_attention(qq, k, v, is_causal=True, scale=scale)
        else:
            mask = torch.arange(kl)[None, :] <= (kl - ql + torch.arange(ql))[:, None]
            ref = F.scaled_dot_product_attention(qq, k, v, attn_mask=mask, scale=scale)
        np.testing.assert_allclose(ours[qs:qe], ref.transpose(0, 1).numpy(), rtol=1e-10,
                                   atol=1e-12)
        if ql > 1 and kl > ql:  # planted mistake: a top-left aligned mask differs
            wrong_mask = torch.arange(kl)[None, :] <= torch.arange(ql)[:, None]
            wrong = F.scaled_dot_product_attention(qq, k, v, attn_mask=wrong_mask, scale=scale)
            assert not np.allclose(ours[qs:qe], wrong.transpose(0, 1).numpy(), atol=1e-3)


def test_paged_prefill_decode_case_and_causality():
    q, kc, vc, bt, cu_q, cu_k = _prefill_case(seed=22, q_lens=(1, 1), k_lens=(13, 24))
    lens = np.diff(cu_k)
    pre = oracle.paged_prefill(q, kc, vc, bt, cu_q, cu_k, 0.25)
    dec = oracle.paged_decode(q, kc, vc, bt, lens, 0.25)
    np.testing.assert_allclose(pre, dec, rtol=1e-12, atol=1e-13)
    # causality: changing the keys after query 2's position leaves queries 0..2 unchanged
    q, kc, vc, bt, cu_q, cu_k = _prefill_case(seed=23, q_lens=(6,), k_lens=(10,))
    base = oracle.paged_prefill(q, kc, vc, bt, cu_q, cu_k, 0.25)
    kc2, vc2 = kc.copy(), vc.copy()
    bs = kc.shape[1]
    for t in range(10 - 6 + 3, 10):  # positions after query 2 (at position 6)
        page, slot = bt[0, t // bs], t % bs
        kc2[page, slot] += 5.0
        vc2[page, slot] -= 3.0
    moved = oracle.paged_prefill(q, kc2, vc2, bt, cu_q, cu_k, 0.25)
    np.testing.assert_allclose(moved[:3], base[:3], rtol=1e-12, atol=1e-13)
    assert not np.allclose(moved[3:], base[3:])
    # a query with no visible key (q_len > k_len) gives zeros
    q, kc, vc, bt, cu_q, cu_k = _prefill_case(seed=24, q_lens=(5,), k_lens=(3,))
    z = oracle.paged_prefill(q, kc, vc, bt, cu_q, cu_k, 0.25)
    assert np.array_equal(z[:2], np.zeros_like(z[:2])) and np.abs(z[2:]).sum() > 0


# ---------------------------------------------------------------------------
# dense (varlen) prefill: _prefill_torch_from_tensors, attention_impl.py:624-638
# ---------------------------------------------------------------------------
def _varlen_case(seed=31, q_lens=(5, 1, 9, 4), k_lens=(5, 17, 30, 4), hq=4, hk=2, d=16):
    """Dense keys of several sequences packed back to back, with k_len > q_len for some
    (chunks over a cached prefix) and k_len == q_len for others (whole prompts)."""
    rng = np.random.default_rng(seed)
    cu_q = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(k_lens)]).astype(np.int32)
    q = rng.standard_normal((int(cu_q[-1]), hq, d)).astype(np.float32)
    key = rng.standard_normal((int(cu_k[-1]), hk, d)).astype(np.float32)
    value = rng.standard_normal((int(cu_k[-1]), hk, d)).astype(np.float32)
    return q, key, value, cu_q, cu_k


def test_varlen_prefill_vs_torch_sdpa():
    """Each sequence against float64 torch SDPA over its own dense K/V slice, with the
    end-aligned causal mask (key_offset = k_len - q_len, attention_impl.py:630-636)."""
    q, key, value, cu_q, cu_k = _varlen_case()
    scale = 0.3
    ours = oracle.varlen_prefill(q, key, value, cu_q, cu_k, scale)
    hq, hk = q.shape[1], key.shape[1]
    for i in range(len(cu_q) - 1):
        qs, qe, ks, ke = int(cu_q[i]), int(cu_q[i + 1]), int(cu_k[i]), int(cu_k[i + 1])
        ql, kl = qe - qs, ke - ks
        k = torch.from_numpy(key[ks:ke]).double().repeat_interleave(hq // hk, 1).transpose(0, 1)
        v = torch.from_numpy(value[ks:ke]).double().repeat_interleave(hq // hk, 1).transpose(0, 1)
        qq = torch.from_numpy(q[qs:qe]).double().transpose(0, 1)
        mask = torch.arange(kl)[None, :] <= (kl - ql + torch.arange(ql))[:, None]
        ref = F.scaled_dot_product_attention(qq, k, v, attn_mask=mask, scale=scale)
        np.testing.assert_allclose(ours[qs:qe], ref.transpose(0, 1).numpy(), rtol=1e-10,
                                   atol=1e-12)
    # non-causal: every query sees its sequence's whole slice
    full = oracle.varlen_prefill(q, key, value, cu_q, cu_k, scale, causal=False)
    i = 2
    qs, qe, ks, ke = int(cu_q[i]), int(cu_q[i + 1]), int(cu_k[i]), int(cu_k[i + 1])
    k = torch.from_numpy(key[ks:ke]).double().repeat_interleave(hq // hk, 1).transpose(0, 1)
    v = torch.from_numpy(value[ks:ke]).double().repeat_interleave(hq // hk, 1).transpose(0, 1)
    qq = torch.from_numpy(q[qs:qe]).double().transpose(0, 1)
    ref = F.scaled_dot_product_attention(qq, k, v, scale=scale)
    np.testing.assert_allclose(full[qs:qe], ref.transpose(0, 1).numpy(), rtol=1e-10, atol=1e-12)


def test_varlen_prefill_equals_paged_prefill_on_scattered_keys():
    """Closed-form layout relation: the same keys scattered into shuffled pages and read
    through a block table give the dense result (varlen == paged)."""
    q, key, value, cu_q, cu_k = _varlen_case(seed=32)
    hk, d = key.shape[1], key.shape[2]
    bs = 8
    k_lens = np.diff(cu_k)
    pages = [(int(n) + bs - 1) // bs for n in k_lens]
    nb = sum(pages) + 3
    rng = np.random.default_rng(5)
    perm = rng.permutation(nb)
    kc = rng.standard_normal((nb, bs, hk, d)).astype(np.float32)  # junk outside the keys
    vc = rng.standard_normal((nb, bs, hk, d)).astype(np.float32)
    bt = np.full((len(k_lens), max(pages)), -1, np.int32)
    off = 0
    for i, n in enumerate(k_lens):
        bt[i, :pages[i]] = perm[off:off + pages[i]]
        off += pages[i]
        for t in range(int(n)):
            kc[bt[i, t // bs], t % bs] = key[cu_k[i] + t]
            vc[bt[i, t // bs], t % bs] = value[cu_k[i] + t]
    dense = oracle.varlen_prefill(q, key, value, cu_q, cu_k, 0.25)
    paged = oracle.paged_prefill(q, kc, vc, bt, cu_q, cu_k, 0.25)
    np.testing.assert_allclose(dense, paged, rtol=1e-12, atol=1e-13)


def test_varlen_prefill_planted_cu_seqlens_swap_is_caught():
    """A plausible slip, slicing Q by cu_seqlens_k and K by cu_seqlens_q, changes the
    result: the checks above would catch an oracle that made it."""
    q, key, value, cu_q, cu_k = _varlen_case(seed=33, q_lens=(3, 6), k_lens=(7, 6))
    good = oracle.varlen_prefill(q, key, value, cu_q, cu_k, 0.25)
    qpad = np.concatenate([q, np.zeros((int(cu_k[-1]) - q.shape[0],) + q.shape[1:], q.dtype)])
    swapped = oracle.varlen_prefill(qpad, key, value, cu_k, cu_q, 0.25)[:q.shape[0]]
    assert not np.allclose(good, swapped, atol=1e-3)


def _masked_scores64(q, key, cu_q, cu_k, i, scale, causal):
    """Scores [hq, q_len, k_len] of sequence i in float64 with -inf where masked
    (end-aligned causal or all keys), by torch's matmul."""
    qs, qe, ks, ke = int(cu_q[i]), int(cu_q[i + 1]), int(cu_k[i]), int(cu_k[i + 1])
    ql, kl = qe - qs, ke - ks
    hq, hk = q.shape[1], key.shape[1]
    k = torch.from_numpy(key[ks:ke]).double().repeat_interleave(hq // hk, 1).transpose(0, 1)
    qq = torch.from_numpy(q[qs:qe]).double().transpose(0, 1)
    sc = torch.matmul(qq, k.transpose(1, 2)) * scale
    if causal:
        mask = torch.arange(kl)[None, :] <= (kl - ql + torch.arange(ql))[:, None]
        sc = sc.masked_fill(~mask, float("-inf"))
    return sc


@pytest.mark.parametrize("causal", [True, False])
def test_varlen_prefill_lse_vs_torch_logsumexp(causal):
    """return_lse: lse[h, cu_q[i] + j] equals torch.logsumexp (float64) of query j's
    visible scaled scores; a chunk longer than its keys (causal) has rows with no visible
    key, whose lse is -inf (and whose output row is zero)."""
    q, key, value, cu_q, cu_k = _varlen_case(seed=41, q_lens=(5, 1, 9, 6), k_lens=(5, 17, 30, 4))
    scale = 0.3
    out, lse = oracle.varlen_prefill(q, key, value, cu_q, cu_k, scale, causal=causal,
                                     return_lse=True)
    assert lse.shape == (q.shape[1], q.shape[0])
    np.testing.assert_array_equal(out, oracle.varlen_prefill(q, key, value, cu_q, cu_k, scale,
                                                             causal=causal))
    for i in range(len(cu_q) - 1):
        qs, qe = int(cu_q[i]), int(cu_q[i + 1])
        ref = torch.logsumexp(_masked_scores64(q, key, cu_q, cu_k, i, scale, causal), dim=-1)
        np.testing.assert_allclose(lse[:, qs:qe], ref.numpy(), rtol=1e-12, atol=1e-12)
    if causal:  # sequence 3: 6 queries over 4 keys, its first two see nothing
        assert np.isneginf(lse[:, int(cu_q[3]):int(cu_q[3]) + 2]).all()
        assert (out[int(cu_q[3]):int(cu_q[3]) + 2] == 0).all()
    # Planted mistakes a kernel could make are caught: the log in base 2, or the
    # unscaled scores.
    fin = np.isfinite(lse)
    ln2 = np.where(fin, lse / np.log(2.0), 0.0)
    assert not np.allclose(ln2[fin], lse[fin], atol=1e-3)
    bad = oracle.varlen_prefill(q, key, value, cu_q, cu_k, 1.0, causal=causal, return_lse=True)[1]
    assert not np.allclose(bad[fin], lse[fin], atol=1e-3)


def test_varlen_prefill_lse_merge_of_key_halves_is_whole():
    """Attention over a key set split in two (non-causal, the MLA context-chunk form),
    each half returning (out, lse), merged by merge_attn_states, equals attention over
    the whole set, and the merged lse equals the whole lse."""
    q, key, value, cu_q, cu_k = _varlen_case(seed=42, q_lens=(7, 3), k_lens=(20, 11))
    scale = 0.25
    whole, whole_lse = oracle.varlen_prefill(q, key, value, cu_q, cu_k, scale, causal=False,
                                             return_lse=True)
    halves = []
    for part in (0, 1):
        ks, vs, cuk = [], [], [0]
        for i in range(len(cu_k) - 1):
            a, b = int(cu_k[i]), int(cu_k[i + 1])
            mid = (a + b) // 2
            lo, hi = (a, mid) if part == 0 else (mid, b)
            ks.append(key[lo:hi])
            vs.append(value[lo:hi])
            cuk.append(cuk[-1] + hi - lo)
        halves.append(oracle.varlen_prefill(q, np.concatenate(ks), np.concatenate(vs), cu_q,
                                            np.array(cuk, np.int32), scale, causal=False,
                                            return_lse=True))
    (o0, l0), (o1, l1) = halves
    merged, merged_lse = oracle.merge_attn_states(o0, l0.astype(np.float32), o1,
                                                  l1.astype(np.float32), "f32")
    np.testing.assert_allclose(merged, whole, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(merged_lse, whole_lse, rtol=1e-6, atol=1e-6)


def test_varlen_prefill_value_head_size_differs_vs_torch_sdpa():
    """MLA prefill shapes: query / key head 24 and value head 16 (192 / 128 scaled down):
    against float64 torch SDPA, which takes a value of its own head size."""
    rng = np.random.default_rng(43)
    q_lens, k_lens, hq, hk, d, dv = (4, 9), (4, 13), 4, 4, 24, 16
    cu_q = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(k_lens)]).astype(np.int32)
    q = rng.standard_normal((int(cu_q[-1]), hq, d)).astype(np.float32)
    key = rng.standard_normal((int(cu_k[-1]), hk, d)).astype(np.float32)
    value = rng.standard_normal((int(cu_k[-1]), hk, dv)).astype(np.float32)
    for causal in (True, False):
        out = oracle.varlen_prefill(q, key, value, cu_q, cu_k, 0.2, causal=causal)
        assert out.shape == (q.shape[0], hq, dv)
        for i in range(2):
            qs, qe, ks, ke = int(cu_q[i]), int(cu_q[i + 1]), int(cu_k[i]), int(cu_k[i + 1])
            ql, kl = qe - qs, ke - ks
            qq = torch.from_numpy(q[qs:qe]).double().transpose(0, 1)
            k = torch.from_numpy(key[ks:ke]).double().transpose(0, 1)
            v = torch.from_numpy(value[ks:ke]).double().transpose(0, 1)
            mask = (torch.arange(kl)[None, :] <= (kl - ql + torch.arange(ql))[:, None]
                    if causal else None)
            ref = F.scaled_dot_product_attention(qq, k, v, attn_mask=mask, scale=0.2)
            np.testing.assert_allclose(out[qs:qe], ref.transpose(0, 1).numpy(), rtol=1e-10,
                                       atol=1e-12)


# ---------------------------------------------------------------------------
# the reference's torch decode path (the CPU baseline leg), oracle/torch_path.py
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_decode_torch_matches_oracle(dtype, tol):
    """oracle.torch_path.decode_torch (what bench.py's cpu_baseline times) against the
    pinned numpy paged_decode: float32 to rounding, bf16 within the bf16 bar."""
    from oracle.torch_path import decode_torch

    q, kc, vc, bt, lens = _decode_case(b=5, hq=8, hk=2, d=32, bs=8, nb=64, seed=3)
    out = decode_torch(torch.from_numpy(q).to(dtype), torch.from_numpy(kc).to(dtype),
                       torch.from_numpy(vc).to(dtype), torch.from_numpy(lens),
                       torch.from_numpy(bt), 0.2)
    qr, kr, vr = (oracle.round_to(a, "bf16") if dtype == torch.bfloat16 else a
                  for a in (q, kc, vc))
    ref = oracle.paged_decode(qr, kr, vr, bt, lens, 0.2)
    np.testing.assert_allclose(out.float().numpy(), ref, rtol=tol, atol=tol)


def test_decode_torch_fp8_matches_oracle():
    """The torch path on fp8 pages (dequantised per kv head after the gather) against
    the numpy paged_decode on the same bytes and scales, within the fp8 bar."""
    from oracle.torch_path import decode_torch

    q, kc, vc, bt, lens = _decode_case(b=4, hq=8, hk=2, d=32, bs=8, nb=64, seed=4)
    ks = np.array([0.05, 0.09], np.float32)
    vs = np.array([0.02, 0.07], np.float32)
    k8 = (torch.from_numpy(kc) / torch.from_numpy(ks).view(1, 1, 2, 1)).to(torch.float8_e4m3fn)
    v8 = (torch.from_numpy(vc) / torch.from_numpy(vs).view(1, 1, 2, 1)).to(torch.float8_e4m3fn)
    qb = torch.from_numpy(q).to(torch.bfloat16)
    out = decode_torch(qb, k8, v8, torch.from_numpy(lens), torch.from_numpy(bt), 0.2,
                       k_scale=torch.from_numpy(ks), v_scale=torch.from_numpy(vs))
    ref = oracle.paged_decode(qb.float().numpy(), k8.view(torch.uint8).numpy(),
                              v8.view(torch.uint8).numpy(), bt, lens, 0.2, ks, vs)
    np.testing.assert_allclose(out.float().numpy(), ref, rtol=3e-2, atol=3e-2)


@pytest.mark.parametrize("window_left", [0, 3, 9, 40])
def test_paged_prefill_window_and_sinks(window_left):
    """Prefill with a sliding window and sinks: one-query chunks equal the decode
    (itself pinned against SDPA); a multi-query chunk equals torch's softmax over the
    masked scores with the sink as one more column; keys before a query's window
    start do not move its output and keys inside do."""
    q, kc, vc, bt, cu_q, cu_k = _prefill_case(seed=25, q_lens=(1, 1), k_lens=(13, 24))
    sinks = np.linspace(-1.0, 1.5, q.shape[1])
    pre = oracle.paged_prefill(q, kc, vc, bt, cu_q, cu_k, 0.25, window_left=window_left,
                               sinks=sinks)
    dec = oracle.paged_decode(q, kc, vc, bt, np.diff(cu_k), 0.25, window_left=window_left,
                              sinks=sinks)
    np.testing.assert_allclose(pre, dec, rtol=1e-12, atol=1e-13)
    q, kc, vc, bt, cu_q, cu_k = _prefill_case(seed=26, q_lens=(7,), k_lens=(19,))
    out = oracle.paged_prefill(q, kc, vc, bt, cu_q, cu_k, 0.25, window_left=window_left,
                               sinks=sinks)
    hq, hk = q.shape[1], kc.shape[2]
    ks = torch.from_numpy(oracle.gather_seq(kc, bt[0], 19)).double()[:, torch.arange(hq) // (hq // hk)]
    vs = torch.from_numpy(oracle.gather_seq(vc, bt[0], 19)).double()[:, torch.arange(hq) // (hq // hk)]
    qt = torch.from_numpy(q).double()  # [7, Hq, D]
    sc = torch.einsum("jhd,thd->hjt", qt, ks) * 0.25
    pos = torch.arange(7) + 12
    t = torch.arange(19)
    mask = (t[None, :] <= pos[:, None]) & (t[None, :] >= pos[:, None] - window_left)
    sc = sc.masked_fill(~mask[None], float("-inf"))
    sink = torch.from_numpy(sinks).double()[:, None, None].expand(hq, 7, 1)
    p = torch.softmax(torch.cat([sc, sink], -1), -1)[..., :19]
    ref = torch.einsum("hjt,thd->jhd", p, vs).numpy()
    np.testing.assert_allclose(out, ref, rtol=1e-10, atol=1e-12)
    # locality: key 12 + 3 - window_left - 1 is before query 3's window, key pos_3 is inside
    kc2, vc2 = kc.copy(), vc.copy()
    bs = kc.shape[1]
    before = 12 + 3 - window_left - 1
    if before >= 0:
        page, slot = bt[0, before // bs], before % bs
        kc2[page, slot] += 5.0
        vc2[page, slot] -= 3.0
        moved = oracle.paged_prefill(q, kc2, vc2, bt, cu_q, cu_k, 0.25, window_left=window_left,
                                     sinks=sinks)
        np.testing.assert_allclose(moved[3:], out[3:], rtol=1e-12, atol=1e-13)
    page, slot = bt[0, 15 // bs], 15 % bs
    kc2[page, slot] += 5.0
    moved = oracle.paged_prefill(q, kc2, vc2, bt, cu_q, cu_k, 0.25, window_left=window_left,
                                 sinks=sinks)
    assert not np.allclose(moved[3], out[3])


# ---------------------------------------------------------------------------
# merge_attn_states
# ---------------------------------------------------------------------------
def _halves(seed=11, t=5, h=3, d=16, n=40, cut=17):
    """Per (token, head): attention of a query over n keys, and over the keys
    [0, cut) and [cut, n) separately, with natural-log lse, from torch in float64."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(t, h, 1, d, generator=g, dtype=torch.float64)
    k = torch.randn(t, h, n, d, generator=g, dtype=torch.float64)
    v = torch.randn(t, h, n, d, generator=g, dtype=torch.float64)
    sc = 0.4

    def part(lo, hi):
        o = F.scaled_dot_product_attention(q, k[:, :, lo:hi], v[:, :, lo:hi], scale=sc)[:, :, 0]
        lse = torch.logsumexp((q @ k[:, :, lo:hi].transpose(-1, -2))[:, :, 0] * sc, dim=-1)
        return o.numpy(), lse.T.contiguous().numpy()  # o [T, H, D], lse [H, T]

    return part(0, cut), part(cut, n), part(0, n)


def test_merge_attn_states_equals_attention_over_the_union():
    (po, pl), (so, sl), (whole, whole_lse) = _halves()
    out, out_lse = oracle.merge_attn_states(po, pl, so, sl, "f32")
    np.testing.assert_allclose(out, whole, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out_lse, whole_lse, rtol=1e-6)
    # planted mistake: the prefix weight applied to the suffix is caught
    m = np.maximum(pl, sl).T[..., None]
    wp, ws = np.exp(pl.T[..., None] - m), np.exp(sl.T[..., None] - m)
    wrong = (po * ws + so * wp) / (wp + ws)
    assert not np.allclose(wrong, whole, atol=1e-3), "planted mistake (swapped weights) not caught"


def test_merge_attn_states_special_cases():
    (po, pl), (so, sl), _ = _halves(seed=12, t=6, h=2)
    pl, sl = pl.astype(np.float32), sl.astype(np.float32)
    pl[0, 0] = -np.inf            # empty prefix -> the suffix
    sl[0, 1] = -np.inf            # empty suffix -> the prefix
    pl[1, 2] = sl[1, 2] = -np.inf  # both empty -> prefix rows, lse -inf
    pl[1, 3] = np.inf             # +inf is read as -inf (as empty)
    out, out_lse = oracle.merge_attn_states(po, pl, so, sl, "f32", prefill_tokens_with_context=5)
    np.testing.assert_allclose(out[0, 0], so[0, 0], rtol=1e-6)
    np.testing.assert_allclose(out[1, 0], po[1, 0], rtol=1e-6)
    assert np.array_equal(out[2, 1], po[2, 1].astype(np.float32)) and out_lse[1, 2] == -np.inf
    np.testing.assert_allclose(out[3, 1], so[3, 1], rtol=1e-6)
    assert out_lse[0, 0] == pytest.approx(sl[0, 0], rel=1e-6)
    assert out_lse[1, 3] == pytest.approx(sl[1, 3], rel=1e-6)
    # token 5 >= prefill_tokens_with_context: suffix copied, lse copied
    assert np.array_equal(out[5], so[5].astype(np.float32)) and np.array_equal(out_lse[:, 5], sl[:, 5])
    assert np.isfinite(out).all()
    # bf16: one rounding of the fp32 value
    b, _ = oracle.merge_attn_states(po, pl, so, sl, "bf16")
    f, _ = oracle.merge_attn_states(po, pl, so, sl, "f32")
    mask = np.ones(f.shape[:2], bool)
    mask[2, 1] = False  # copied row, not rounded
    assert np.array_equal(b[mask], oracle.round_to(f[mask], "bf16"))


def test_merge_attn_states_fp8_output():
    """The fp8 output (output_scale): copied rows are torch's own e4m3fn cast of
    value / scale (exact); merged rows are within one e4m3fn step of the fp32 merge /
    scale; values beyond +-448 saturate and NaN becomes 448 (fmin/fmax clamp); a
    planted mistake (multiplying by the scale instead of dividing) is caught."""
    (po, pl), (so, sl), _ = _halves(seed=13, t=6, h=2)
    pl, sl = pl.astype(np.float32), sl.astype(np.float32)
    po = (po * 40).astype(np.float32)
    so = (so * 40).astype(np.float32)
    so[5, 0, 0] = np.nan
    so[5, 0, 1] = 1e6
    scale = 0.25
    codes, lse = oracle.merge_attn_states(po, pl, so, sl, "bf16", prefill_tokens_with_context=5,
                                          output_scale=scale)
    assert codes.dtype == np.uint8
    f32, f_lse = oracle.merge_attn_states(po, pl, so, sl, "f32", prefill_tokens_with_context=5)
    np.testing.assert_array_equal(lse, f_lse)
    dec = oracle.fp8_e4m3fn_decode(codes)
    # copied suffix rows (token 5): torch's cast of the clamped value / scale
    x = torch.from_numpy(so[5] * np.float32(1 / scale)).clamp(-448, 448)
    want = torch.nan_to_num(x, nan=448.0).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(codes[5], want)
    assert dec[5, 0, 0] == 448.0 and dec[5, 0, 1] == 448.0
    # merged rows: within one e4m3fn step (2^-3 relative, 2^-9 absolute below 2^-6)
    ref = np.clip(f32[:5] / scale, -448, 448)
    step = np.maximum(np.abs(ref) * 2.0 ** -3, 2.0 ** -9)
    assert (np.abs(dec[:5] - ref) <= step).all()
    wrong = oracle.fp8_e4m3fn_decode(oracle.fp8_e4m3fn_encode(np.clip(f32[:5] * scale, -448, 448)))
    assert not (np.abs(wrong - ref) <= step).all(), "planted mistake (scale multiplied) not caught"


# ---------------------------------------------------------------------------
# SiLU-and-mul
# ---------------------------------------------------------------------------
def test_silu_and_mul_matches_torch():
    x = oracle.round_to((RNG.standard_normal((64, 2 * 96)) * 4).astype(np.float32), "bf16")
    xt = torch.from_numpy(x).bfloat16()
    ref = (F.silu(xt[:, :96]) * xt[:, 96:]).float().numpy()  # forward_native in bf16
    ours = oracle.silu_and_mul(x, "bf16")
    diff = np.abs(ours - ref)
    assert (diff <= 1e-2 * np.abs(ref) + 1e-6).all()
    assert (ours == ref).mean() > 0.99  # same rounding points: nearly all bit-identical
    np.testing.assert_allclose(oracle.silu_and_mul(np.array([[0.0, 3.0]], np.float32), "f32"), [[0.0]])
    big = oracle.silu_and_mul(np.array([[30.0, 2.0]], np.float32), "f32")
    np.testing.assert_allclose(big, [[60.0]], rtol=1e-6)  # silu(x) -> x for large x


def test_torch_native_paths_match_oracle():
    """The torch restatements bench.py times as CPU baselines (RMSNorm / rotary /
    SiLU forward_native, the store as a scatter) against the pinned numpy oracle on
    the same inputs: fp32 to rounding, the store bit for bit."""
    from oracle import torch_path as tp

    g = torch.Generator().manual_seed(11)
    x = torch.randn(6, 64, generator=g)
    r = torch.randn(6, 64, generator=g)
    w = 1 + 0.1 * torch.randn(64, generator=g)
    out, res = tp.rms_norm_native(x, w, 1e-6, residual=r)
    ref_out, ref_res = oracle.rms_norm(x.numpy(), w.numpy(), 1e-6, "f32", residual=r.numpy())
    np.testing.assert_allclose(out.numpy(), ref_out, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(res.numpy(), ref_res, rtol=0, atol=0)

    cache = oracle.rope_cos_sin_cache(16, 32, 10000.0)
    pos = torch.tensor([0, 3, 31, 7])
    q = torch.randn(4, 2 * 16, generator=g)
    k = torch.randn(4, 1 * 16, generator=g)
    qo, ko = tp.rotary_native(pos, q, k, 16, torch.from_numpy(cache).float())
    rq, rk = oracle.rotary(pos.numpy(), q.numpy(), k.numpy(), 16, cache, True, "f32")
    np.testing.assert_allclose(qo.numpy(), rq, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(ko.numpy(), rk, rtol=1e-5, atol=1e-6)

    key = torch.randn(5, 2, 8, generator=g)
    val = torch.randn(5, 2, 8, generator=g)
    slots = torch.tensor([3, -1, 0, 9, 6])
    kc, vc = torch.zeros(3, 4, 2, 8), torch.zeros(3, 4, 2, 8)
    tp.store_kvcache_torch(key, val, kc, vc, slots)
    kr, vr = np.zeros((3, 4, 2, 8), np.float32), np.zeros((3, 4, 2, 8), np.float32)
    oracle.store_kvcache_(key.numpy(), val.numpy(), kr, vr, slots.numpy())
    assert np.array_equal(kc.numpy(), kr) and np.array_equal(vc.numpy(), vr)

    gu = torch.randn(3, 2 * 24, generator=g)
    np.testing.assert_allclose(tp.silu_and_mul_native(gu).numpy(),
                               oracle.silu_and_mul(gu.numpy(), "f32"), rtol=1e-5, atol=1e-6)
