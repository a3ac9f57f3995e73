"""The drop-in surface (no GPU): candidate files load the way the reference harness
loads them, expose the baseline class names and signatures, carry the same
parameters / buffers, and register opaque custom ops with fake impls.

Reference contract: a candidate lives at tasks/candidate/L1/<stem>.py and defines
the class named like the baseline (fastkernels/bench.py:239-271,
fastkernels/list.py:443-467); bench.py loads baseline weights into it with
load_state_dict(strict=False) (fastkernels/bench.py:2177).
"""
from __future__ import annotations

import importlib.util
import inspect
import math
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle

ROOT = Path(__file__).resolve().parents[1]
CAND = ROOT / "fastkernels_amd" / "candidate" / "L1"

# stem -> (class name, __init__ parameters, forward parameters) of the reference baseline
# (fastkernels/tasks/baseline/L1/<stem>.py); None = no __init__ of its own (nn.Module's).
CONTRACT = {
    "rms_norm": ("RMSNorm", ["hidden_size", "eps", "elementwise_affine"], ["x", "residual"]),
    "rotary_emb": ("RotaryEmbedding",
                   ["head_dim", "max_position_embeddings", "rope_theta", "rope_scaling_factor",
                    "rope_low_freq_factor", "rope_high_freq_factor",
                    "rope_original_max_position_embeddings", "is_neox_style"],
                   ["positions", "query", "key"]),
    "store_kvcache": ("StoreKVCache", None, ["key", "value", "k_cache", "v_cache", "slot_mapping"]),
    "flash_attn_decode": ("FlashAttnDecode", ["num_heads", "num_kv_heads", "head_dim", "page_size"],
                          ["q", "k_cache", "v_cache", "cache_seqlens", "kwargs"]),
    "silu_and_mul": ("SiluAndMul", [], ["x"]),
    "flash_attn_prefill": ("FlashAttnPrefill", ["num_heads", "num_kv_heads", "head_dim"],
                           ["q", "k", "v", "cu_seqlens_q", "cu_seqlens_k", "max_seqlen_q",
                            "max_seqlen_k", "kwargs"]),
    "flash_attn_varlen": ("FlashAttnVarlen", None,
                          ["q", "k", "v", "cu_seqlens_q", "cu_seqlens_k", "max_seqlen_q",
                           "max_seqlen_k", "softmax_scale", "causal", "return_softmax_lse"]),
    "merge_attn_states": ("MergeAttnStates", None,
                          ["output", "prefix_output", "prefix_lse", "suffix_output", "suffix_lse",
                           "output_lse"]),
}


def load_by_path(stem: str):
    """As the reference harness does: spec_from_file_location on the bare file."""
    spec = importlib.util.spec_from_file_location(f"_fk_candidate_L1_{stem}", CAND / f"{stem}.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.mark.parametrize("stem", sorted(CONTRACT))
def test_candidate_class_and_signatures(stem):
    cls_name, init_params, fwd_params = CONTRACT[stem]
    cls = getattr(load_by_path(stem), cls_name)
    assert issubclass(cls, torch.nn.Module)
    fwd = [p for p in inspect.signature(cls.forward).parameters if p != "self"]
    if init_params is None:
        assert "__init__" not in cls.__dict__
    else:
        init = [p for p in inspect.signature(cls.__init__).parameters if p != "self"]
        assert init == init_params
    assert fwd == fwd_params


def test_attention_candidates_refuse_unbuilt_head_sizes_at_construction():
    """A head size the kernels are not built for is refused by the constructor, not at
    the first forward: decode runs at 64 / 128 / 256; prefill also at 32, 72, 80 and 96
    (Qwen-VL vision encoders: 1280 / 16 = 80, L2/vision_attention.py:32,39)."""
    dec = load_by_path("flash_attn_decode").FlashAttnDecode
    pre = load_by_path("flash_attn_prefill").FlashAttnPrefill
    for d in (64, 128, 256):
        dec(8, 2, d)
    for d in (80, 96, 192, 512):
        with pytest.raises(NotImplementedError, match="head_dim"):
            dec(8, 2, d)
    for d in (32, 64, 72, 80, 96, 128, 256):
        assert pre(16, 16, d).head_dim == d
    for d in (48, 192, 512):
        with pytest.raises(NotImplementedError, match="head_dim"):
            pre(8, 2, d)


def test_flash_attn_varlen_refuses_unbuilt_head_sizes():
    """FlashAttnVarlen takes no head size at construction: an unbuilt (query / key,
    value) pair is refused at forward, before anything runs (CPU tensors here)."""
    cls = load_by_path("flash_attn_varlen").FlashAttnVarlen
    cu = torch.tensor([0, 4], dtype=torch.int32)
    for d, dv in ((48, 48), (128, 64), (192, 192)):
        q = torch.zeros(4, 2, d, dtype=torch.bfloat16)
        v = torch.zeros(4, 2, dv, dtype=torch.bfloat16)
        with pytest.raises(NotImplementedError, match="head sizes"):
            cls()(q, q, v, cu, cu, 4, 4, 0.1, True, True)


def test_merge_attn_states_function_signature():
    """merge_attn_states.py:32-41: the module-level function keeps the reference's arguments."""
    fn = load_by_path("merge_attn_states").merge_attn_states
    assert list(inspect.signature(fn).parameters) == [
        "output", "prefix_output", "prefix_lse", "suffix_output", "suffix_lse", "output_lse",
        "prefill_tokens_with_context", "output_scale"]


def test_candidate_loads_in_a_fresh_interpreter_without_repo_on_path(tmp_path):
    """A file-path import from another working directory still finds the package."""
    code = ("import importlib.util, sys; "
            f"spec = importlib.util.spec_from_file_location('c', r'{CAND / 'rms_norm.py'}'); "
            "m = importlib.util.module_from_spec(spec); spec.loader.exec_module(m); "
            "print(m.RMSNorm(64).weight.shape[0])")
    out = subprocess.run([sys.executable, "-c", code], cwd=tmp_path, capture_output=True,
                         text=True, timeout=240)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip().endswith("64")


def test_rmsnorm_parameters_and_state_dict():
    RMSNorm = load_by_path("rms_norm").RMSNorm
    m = RMSNorm(4096)
    assert list(m.state_dict()) == ["weight"] and torch.equal(m.weight.data, torch.ones(4096))
    w = torch.randn(4096)
    m.load_state_dict({"weight": w}, strict=False)
    assert torch.equal(m.weight.data, w)
    assert list(RMSNorm(64, elementwise_affine=False).state_dict()) == []


def test_rotary_cache_matches_reference_construction():
    RotaryEmbedding = load_by_path("rotary_emb").RotaryEmbedding
    m = RotaryEmbedding(128, 4097, 1e6)
    assert m.cos_sin_cache.dtype == torch.float32 and tuple(m.cos_sin_cache.shape) == (4097, 128)
    # float32 angles t * inv_freq (as the reference forms them) carry up to half an ulp
    # of 4096, 2.4e-4, so cos/sin agree to that; the first positions agree to 1e-6.
    ref = oracle.rope_cos_sin_cache(128, 4097, 1e6)
    np.testing.assert_allclose(m.cos_sin_cache.numpy(), ref, atol=5e-4)
    np.testing.assert_allclose(m.cos_sin_cache.numpy()[:16], ref[:16], atol=1e-6)
    assert "cos_sin_cache" not in m.state_dict()  # non-persistent, as the reference


def test_gemma4_proportional_rotary_cache():
    """Gemma4ProportionalRotaryEmbedding (rotary_emb.py:194-230): the reference's
    constructor, a [max_pos, head_dim] cache whose rotated pairs use exponents over the
    full head dim and whose remaining pairs are identity (cos 1, sin 0); dividing by
    rotary_dim instead would be caught."""
    mod = load_by_path("rotary_emb")
    G = mod.Gemma4ProportionalRotaryEmbedding
    assert issubclass(G, mod.RotaryEmbedding)
    params = [p for p in inspect.signature(G.__init__).parameters if p != "self"]
    assert params == ["head_dim", "rotary_dim", "max_position_embeddings", "rope_theta"]
    m = G(256, 64, 1000, 1e6)
    c = m.cos_sin_cache
    assert c.dtype == torch.float32 and tuple(c.shape) == (1000, 256)
    cos, sin = c[:, :128].double(), c[:, 128:].double()
    assert torch.equal(cos[:, 32:], torch.ones_like(cos[:, 32:]))
    assert torch.equal(sin[:, 32:], torch.zeros_like(sin[:, 32:]))
    i = torch.arange(32, dtype=torch.float64)
    t = torch.arange(1000, dtype=torch.float64)[:, None]
    ang = t * (1e6 ** (-2 * i / 256))[None]
    torch.testing.assert_close(cos[:, :32], torch.cos(ang), atol=5e-4, rtol=0)
    torch.testing.assert_close(sin[:, :32], torch.sin(ang), atol=5e-4, rtol=0)
    wrong = t * (1e6 ** (-2 * i / 64))[None]
    assert not torch.allclose(cos[:, :32], torch.cos(wrong), atol=1e-2)
    assert m.is_neox_style and m.head_dim == 256 and "cos_sin_cache" not in m.state_dict()


def test_store_kvcache_hnd_class():
    """StoreKVCacheHND(page_size).forward(key, value, k_cache, v_cache, slot_mapping)
    (store_kvcache.py:85-99); CPU tensors are refused, not computed."""
    H = load_by_path("store_kvcache").StoreKVCacheHND
    assert [p for p in inspect.signature(H.__init__).parameters if p != "self"] == ["page_size"]
    assert [p for p in inspect.signature(H.forward).parameters if p != "self"] == \
        ["key", "value", "k_cache", "v_cache", "slot_mapping"]
    m = H(16)
    assert m.page_size == 16
    kv = torch.zeros(3, 2, 128, dtype=torch.bfloat16)
    cache = torch.zeros(4, 2, 16, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        m(kv, kv, cache, cache, torch.zeros(3, dtype=torch.int64))


def test_rotary_llama31_scaling():
    """Llama-3.1 frequency scaling (rotary_emb.py:44-68): high frequencies kept, low
    frequencies divided by the factor, a smooth blend in between."""
    RotaryEmbedding = load_by_path("rotary_emb").RotaryEmbedding
    d, theta, factor, lo, hi, orig = 128, 5e5, 8.0, 1.0, 4.0, 8192
    m = RotaryEmbedding(d, 16, theta, factor, lo, hi, orig)
    inv = 1.0 / theta ** (np.arange(0, d, 2) / d)
    wl = 2 * math.pi / inv
    expect = np.where(wl < orig / hi, inv,
                      np.where(wl > orig / lo, inv / factor,
                               (1 - (orig / wl - lo) / (hi - lo)) * inv / factor
                               + (orig / wl - lo) / (hi - lo) * inv))
    got_inv = m.cos_sin_cache[1, d // 2:].numpy()  # sin(1 * inv_freq)
    np.testing.assert_allclose(np.arcsin(got_inv), expect, rtol=1e-5, atol=1e-7)
    assert (expect < inv).any() and (expect == inv).any()


def test_custom_ops_registered_with_fake_impls():
    from fastkernels_amd import ops  # noqa: F401  (registers the library)

    for name in ("rmsnorm", "fused_add_rmsnorm", "rotary_embedding", "store_kvcache",
                 "paged_decode", "silu_and_mul"):
        assert hasattr(torch.ops.fastkernels_amd, name)
    x = torch.empty(8, 2 * 64, device="meta", dtype=torch.bfloat16)
    out = torch.empty(8, 64, device="meta", dtype=torch.bfloat16)
    torch.ops.fastkernels_amd.silu_and_mul(out, x)  # Meta impl: no kernel, no error
    q = torch.empty(4, 8, 128, device="meta", dtype=torch.bfloat16)
    torch.ops.fastkernels_amd.fused_add_rmsnorm(q, q, torch.empty(128, device="meta",
                                                                  dtype=torch.bfloat16), 1e-6)


def test_flash_attn_decode_argument_errors():
    """Unknown kwargs and malformed sinks are rejected before any launch; CPU tensors
    are refused (no CPU fallback), with or without a window."""
    FlashAttnDecode = load_by_path("flash_attn_decode").FlashAttnDecode
    m = FlashAttnDecode(32, 8, 128, page_size=256)
    q = torch.zeros(2, 32, 128, dtype=torch.bfloat16)
    kc = torch.zeros(4, 256, 8, 128, dtype=torch.bfloat16)
    lens, bt = torch.ones(2, dtype=torch.int32), torch.zeros(2, 1, dtype=torch.int32)
    with pytest.raises(TypeError):
        m(q, kc, kc, lens, block_table=bt, bogus=1)
    with pytest.raises(ValueError, match="s_aux"):
        m(q, kc, kc, lens, block_table=bt, s_aux=torch.zeros(7))
    with pytest.raises(RuntimeError, match="GPU"):
        m(q, kc, kc, lens, block_table=bt, window_size=(128, 0))


def test_flash_attn_decode_engine_hooks():
    """What the reference engine does with its decode ops works on the candidate:
    group them by (heads, kv heads, head dim, window) and share the lead's buffers
    (engine.py:1538-1550, fa_utils.py:108-118), skip the FA3 scheduler refresh for
    an op whose fa_version is not 3 (fa_utils.py:127-145), toggle
    _force_graph_splits (jamba_engine.py:846-856), and set _window_size from the
    layer's sliding window (attention_impl.py:242-244, :282)."""
    FlashAttnDecode = load_by_path("flash_attn_decode").FlashAttnDecode
    ref_pre = ["max_batch_size", "device"]
    pre = [p for p in inspect.signature(FlashAttnDecode.preallocate).parameters if p != "self"]
    assert pre[:2] == ref_pre
    upd = [p for p in inspect.signature(FlashAttnDecode.update_scheduler_metadata).parameters
           if p != "self"]
    assert upd == ["cache_seqlens", "max_seqlen_k", "qkv_dtype", "window_size", "max_seqlen_q"]
    ops_ = [FlashAttnDecode(32, 8, 128) for _ in range(3)]
    ops_[2]._window_size = (4095, 0)
    groups = {}
    for op in ops_:
        key = (op.num_heads, op.num_kv_heads, op.head_dim, tuple(getattr(op, "_window_size")))
        groups.setdefault(key, []).append(op)
    assert [len(g) for g in groups.values()] == [2, 1]
    for group in groups.values():
        lead = group[0]
        if not lead.page_size:
            lead.page_size = 256
        lead.preallocate(8, torch.device("cpu"))
        for op in group[1:]:
            op.page_size = lead.page_size
            op._cu_seqlens_q = lead._cu_seqlens_q
            op._sched_buf = lead._sched_buf
            op._sched_meta = lead._sched_meta
        assert torch.equal(lead._cu_seqlens_q, torch.arange(9, dtype=torch.int32))
        assert getattr(lead, "fa_version", 3) != 3  # the FA3 refresh skips it
        lead.update_scheduler_metadata(torch.ones(8, dtype=torch.int32), 4096,
                                       qkv_dtype=torch.bfloat16,
                                       window_size=getattr(lead, "_window_size", (-1, -1)))
    was = ops_[0]._force_graph_splits
    ops_[0]._force_graph_splits = True
    ops_[0]._force_graph_splits = was
    assert ops_[2]._window_size == (4095, 0)


def test_bench_refuses_multi_gpu():
    out = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120)
    assert out.returncode == 2 and "one GPU" in out.stderr
