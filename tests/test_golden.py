"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle reproduces every committed output exactly, so the fixtures and
the oracle pinned by tests/test_oracle.py stay one and the same reference.
GPU: the gfx950 kernels reproduce the committed outputs (bit-exact for the
store, atol=rtol=1e-2 for bf16, 3e-2 for fp8 KV).
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_fixture_set_present():
    names = {p.stem for p in GOLDEN.glob("*.npz")}
    assert {"rmsnorm_h256", "rmsnorm_h200", "rotary_neox", "rotary_gptj", "store_kvcache",
            "paged_decode_bf16", "paged_decode_fp8", "silu_and_mul_d96",
            "silu_and_mul_d13", "merge_attn_states", "paged_prefill_bf16",
            "qk_norm_rope", "paged_decode_window_sinks", "paged_prefill_window_sinks"} <= names


@pytest.mark.parametrize("h", [256, 200])
def test_oracle_rmsnorm_golden(h):
    g = load(f"rmsnorm_h{h}")
    o, nr = oracle.rms_norm(g["x"], g["weight"], float(g["eps"]), "bf16", residual=g["residual"])
    assert np.array_equal(o, g["out_fused"]) and np.array_equal(nr, g["new_residual"])
    assert np.array_equal(oracle.rms_norm(g["x"], g["weight"], float(g["eps"]), "bf16"),
                          g["out_plain"])


@pytest.mark.parametrize("style", ["neox", "gptj"])
def test_oracle_rotary_golden(style):
    g = load(f"rotary_{style}")
    q, k = oracle.rotary(g["positions"], g["q"], g["k"], 64, g["cos_sin"], style == "neox", "bf16")
    assert np.array_equal(q, g["out_q"]) and np.array_equal(k, g["out_k"])


def test_oracle_store_golden():
    g = load("store_kvcache")
    z = np.zeros_like(g["k_cache"])
    k, v = oracle.store_kvcache(g["key"], g["value"], z, z, g["slot_mapping"])
    assert np.array_equal(k, g["k_cache"]) and np.array_equal(v, g["v_cache"])


@pytest.mark.parametrize("kind", ["bf16", "fp8"])
def test_oracle_decode_golden(kind):
    g = load(f"paged_decode_{kind}")
    out = oracle.paged_decode(g["q"], g["k_cache"], g["v_cache"], g["block_tables"], g["ctx_lens"],
                              float(g["scale"]), g.get("k_scale"), g.get("v_scale"))
    assert np.array_equal(out.astype(np.float32), g["out"])


@pytest.mark.parametrize("d", [96, 13])
def test_oracle_silu_golden(d):
    g = load(f"silu_and_mul_d{d}")
    assert np.array_equal(oracle.silu_and_mul(g["x"], "bf16"), g["out"])


def test_oracle_merge_golden():
    g = load("merge_attn_states")
    o, lse = oracle.merge_attn_states(g["prefix"], g["prefix_lse"], g["suffix"], g["suffix_lse"],
                                      "bf16", int(g["prefill_tokens"]))
    assert np.array_equal(o, g["out"]) and np.array_equal(lse, g["out_lse"])


def test_oracle_prefill_golden():
    g = load("paged_prefill_bf16")
    out = oracle.paged_prefill(g["q"], g["k_cache"], g["v_cache"], g["block_tables"],
                               g["cu_seqlens_q"], g["cu_seqlens_k"], float(g["scale"]))
    assert np.array_equal(out.astype(np.float32), g["out"])


def test_oracle_window_sinks_golden():
    """Window + sinks fixtures, on the inputs of the plain decode / prefill fixtures."""
    g, w = load("paged_decode_bf16"), load("paged_decode_window_sinks")
    out = oracle.paged_decode(g["q"], g["k_cache"], g["v_cache"], g["block_tables"], g["ctx_lens"],
                              float(g["scale"]), window_left=int(w["window_left"]),
                              sinks=w["sinks"])
    assert np.array_equal(out.astype(np.float32), w["out"])
    g, w = load("paged_prefill_bf16"), load("paged_prefill_window_sinks")
    out = oracle.paged_prefill(g["q"], g["k_cache"], g["v_cache"], g["block_tables"],
                               g["cu_seqlens_q"], g["cu_seqlens_k"], float(g["scale"]),
                               window_left=int(w["window_left"]), sinks=w["sinks"])
    assert np.array_equal(out.astype(np.float32), w["out"])


def test_oracle_qk_norm_rope_golden():
    g = load("qk_norm_rope")
    qn = oracle.rms_norm(g["q"].reshape(4, 4, 64), g["q_weight"], float(g["eps"]), "bf16")
    kn = oracle.rms_norm(g["k"].reshape(4, 2, 64), g["k_weight"], float(g["eps"]), "bf16")
    q, k = oracle.rotary(g["positions"], qn.reshape(4, -1), kn.reshape(4, -1), 64, g["cos_sin"],
                         True, "bf16")
    assert np.array_equal(q, g["out_q"]) and np.array_equal(k, g["out_k"])


# ---------------------------------------------------------------------------
# GPU kernels against the same fixtures
# ---------------------------------------------------------------------------
def _t(a, dev, dtype=None):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t.to(dtype) if dtype is not None else t


def _close(got, ref, tol):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    assert np.isfinite(got).all()
    bad = np.abs(got - ref) > tol + tol * np.abs(ref)
    assert not bad.any(), f"{int(bad.sum())} elements outside {tol}; max err {np.abs(got - ref).max()}"


@pytest.mark.gpu
def test_gpu_golden_all(cuda):
    import torch

    from fastkernels_amd import ops

    bf = torch.bfloat16
    f32 = lambda t: t.float().cpu().numpy()
    for h in (256, 200):
        g = load(f"rmsnorm_h{h}")
        x, r, w = _t(g["x"], cuda, bf), _t(g["residual"], cuda, bf), _t(g["weight"], cuda, bf)
        out = torch.empty_like(x)
        ops.rms_norm(out, x, w, float(g["eps"]))
        ops.fused_add_rms_norm(x, r, w, float(g["eps"]))
        torch.cuda.synchronize()
        _close(f32(out), g["out_plain"], 1e-2)
        _close(f32(x), g["out_fused"], 1e-2)
        assert np.array_equal(f32(r), g["new_residual"])
    for style in ("neox", "gptj"):
        g = load(f"rotary_{style}")
        q, k = _t(g["q"], cuda, bf), _t(g["k"], cuda, bf)
        ops.rotary_embedding(_t(g["positions"], cuda), q, k, 64, _t(g["cos_sin"], cuda),
                             style == "neox")
        torch.cuda.synchronize()
        _close(f32(q), g["out_q"], 1e-2)
        _close(f32(k), g["out_k"], 1e-2)
    g = load("store_kvcache")
    kc = torch.zeros(g["k_cache"].shape, dtype=torch.int16, device=cuda).view(bf)
    vc = torch.zeros_like(kc)
    ops.store_kvcache(_t(g["key"], cuda).view(bf), _t(g["value"], cuda).view(bf), kc, vc,
                      _t(g["slot_mapping"], cuda))
    torch.cuda.synchronize()
    assert np.array_equal(kc.view(torch.int16).cpu().numpy(), g["k_cache"])
    assert np.array_equal(vc.view(torch.int16).cpu().numpy(), g["v_cache"])
    for kind, tol in (("bf16", 1e-2), ("fp8", 3e-2)):
        g = load(f"paged_decode_{kind}")
        q = _t(g["q"], cuda, bf)
        if kind == "fp8":
            kc = _t(g["k_cache"], cuda).view(torch.float8_e4m3fn)
            vc = _t(g["v_cache"], cuda).view(torch.float8_e4m3fn)
            ks, vs = _t(g["k_scale"], cuda), _t(g["v_scale"], cuda)
        else:
            kc, vc, ks, vs = _t(g["k_cache"], cuda, bf), _t(g["v_cache"], cuda, bf), None, None
        b, hq, d = q.shape
        for splits in (0, 2):
            plan = ops.paged_decode_plan(b, hq, kc.shape[2], d, int(g["ctx_lens"].max()), splits)
            ws = torch.zeros(max(1, plan.workspace_bytes), dtype=torch.uint8, device=cuda)
            out = torch.full_like(q, float("nan"))
            ops.paged_decode(out, q, kc, vc, _t(g["block_tables"], cuda), _t(g["ctx_lens"], cuda),
                             float(g["scale"]), plan.part_tokens, plan.max_parts, ws, ks, vs)
            torch.cuda.synchronize()
            _close(f32(out), g["out"], tol)
    for d in (96, 13):
        g = load(f"silu_and_mul_d{d}")
        x = _t(g["x"], cuda, bf)
        out = torch.empty(x.shape[0], d, dtype=bf, device=cuda)
        ops.silu_and_mul(out, x)
        torch.cuda.synchronize()
        _close(f32(out), g["out"], 1e-2)

    g = load("merge_attn_states")
    po, so = _t(g["prefix"], cuda, bf), _t(g["suffix"], cuda, bf)
    pl, sl = _t(g["prefix_lse"], cuda), _t(g["suffix_lse"], cuda)
    mo, ml = torch.empty_like(po), torch.empty_like(pl)
    ops.merge_attn_states(mo, po, pl, so, sl, ml, int(g["prefill_tokens"]))
    torch.cuda.synchronize()
    _close(f32(mo), g["out"], 1e-2)
    fin = np.isfinite(g["out_lse"])
    assert np.array_equal(np.isneginf(ml.cpu().numpy()), np.isneginf(g["out_lse"]))
    _close(ml.cpu().numpy()[fin], g["out_lse"][fin], 1e-5)

    g = load("paged_prefill_bf16")
    q = _t(g["q"], cuda, bf)
    out = torch.full_like(q, float("nan"))
    ops.paged_prefill(out, q, _t(g["k_cache"], cuda, bf), _t(g["v_cache"], cuda, bf),
                      _t(g["block_tables"], cuda), _t(g["cu_seqlens_q"], cuda),
                      _t(g["cu_seqlens_k"], cuda), int(np.diff(g["cu_seqlens_q"]).max()),
                      float(g["scale"]))
    torch.cuda.synchronize()
    _close(f32(out), g["out"], 1e-2)
    w = load("paged_prefill_window_sinks")
    out = torch.full_like(q, float("nan"))
    ops.paged_prefill(out, q, _t(g["k_cache"], cuda, bf), _t(g["v_cache"], cuda, bf),
                      _t(g["block_tables"], cuda), _t(g["cu_seqlens_q"], cuda),
                      _t(g["cu_seqlens_k"], cuda), int(np.diff(g["cu_seqlens_q"]).max()),
                      float(g["scale"]), window_left=int(w["window_left"]),
                      sinks=_t(w["sinks"], cuda))
    torch.cuda.synchronize()
    _close(f32(out), w["out"], 1e-2)

    g, w = load("paged_decode_bf16"), load("paged_decode_window_sinks")
    q = _t(g["q"], cuda, bf)
    kc, vc = _t(g["k_cache"], cuda, bf), _t(g["v_cache"], cuda, bf)
    b, hq, d = q.shape
    for splits in (0, 2):
        plan = ops.paged_decode_plan(b, hq, kc.shape[2], d, int(g["ctx_lens"].max()), splits)
        ws = torch.zeros(max(1, plan.workspace_bytes), dtype=torch.uint8, device=cuda)
        out = torch.full_like(q, float("nan"))
        ops.paged_decode(out, q, kc, vc, _t(g["block_tables"], cuda), _t(g["ctx_lens"], cuda),
                         float(g["scale"]), plan.part_tokens, plan.max_parts, ws, None, None,
                         int(w["window_left"]), _t(w["sinks"], cuda))
        torch.cuda.synchronize()
        _close(f32(out), w["out"], 1e-2)

    g = load("qk_norm_rope")
    q, k = _t(g["q"], cuda, bf), _t(g["k"], cuda, bf)
    v = torch.zeros_like(k)
    kc = torch.zeros(2, 16, 2, 64, dtype=bf, device=cuda)
    vc = torch.zeros_like(kc)
    slots = torch.tensor([0, 5, 17, 31], dtype=torch.int64, device=cuda)
    ops.qk_norm_rope_store(_t(g["positions"], cuda), q, k, v, kc, vc, slots, 64,
                           _t(g["cos_sin"], cuda), True, _t(g["q_weight"], cuda, bf),
                           _t(g["k_weight"], cuda, bf), float(g["eps"]))
    torch.cuda.synchronize()
    _close(f32(q), g["out_q"], 1e-2)
    _close(f32(k), g["out_k"], 1e-2)
    assert torch.equal(kc.view(-1, 128)[slots], k)
