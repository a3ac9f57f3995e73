"""The reference bench's acceptance rule and paged-decode input fixer, restated here
(``oracle.compare``, ``oracle.harness.fix_paged_decode``), pinned on the CPU.

The first two tests make the same assertions as the reference's harness test
(tests/test_bench.py:269-316, sections 7a and 7b).  The others pin the rule's
boundaries from the reference code's own definitions (fastkernels/bench.py:141-155,
:1837-1896): at least 99% of elements within atol + rtol*|ref| by the reference
tensor's dtype, a strict ``>`` at the bound, NaN / Inf / all-zero outputs failing
outright, and the first failing leaf deciding.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle.harness import fix_paged_decode


def test_compare_statuses_as_reference_harness():
    rng = np.random.default_rng(0)
    zeros = np.zeros(8, np.float32)
    noise = rng.standard_normal(8).astype(np.float32)
    assert oracle.compare(zeros, zeros, "f32")[0] == oracle.SKIPPED
    assert oracle.compare(noise, noise, "f32")[0] == oracle.PASSED
    assert oracle.compare(zeros, noise, "f32")[0] == oracle.INCORRECT_NUMERICAL
    # zero auxiliary outputs beside a live one still compare (and pass)
    assert oracle.compare((noise, zeros), (noise, zeros), "f32")[0] == oracle.PASSED


def test_fix_paged_decode_as_reference_harness():
    g = torch.Generator().manual_seed(0)
    k = torch.randn(4, 1, 16, 8, generator=g)
    v = torch.randn(4, 1, 16, 8, generator=g)
    k0, v0 = k.clone(), v.clone()
    kw = {"k_cache": k, "v_cache": v, "block_table": torch.zeros(2, 3, dtype=torch.int32),
          "cache_seqlens": torch.zeros(2, dtype=torch.int32), "max_seq_len": 0}
    fix_paged_decode(kw, ("k_cache", "v_cache"), generator=g)
    assert torch.equal(kw["k_cache"], k0) and torch.equal(kw["v_cache"], v0)
    assert int(kw["block_table"].min()) >= 0 and int(kw["block_table"].max()) < 4
    assert int(kw["cache_seqlens"].min()) >= 1
    assert int(kw["max_seq_len"]) == int(kw["cache_seqlens"].max())
    assert kw["block_table"].dtype == torch.int32 and kw["cache_seqlens"].dtype == torch.int32


def test_fix_paged_decode_ranges_and_layouts():
    """Lengths cover [1, max_pages * page_size] and pages cover [0, num_blocks); the
    page size is read from dim -2 (HND, as the reference) or the dim the caller names."""
    g = torch.Generator().manual_seed(1)
    nhd = torch.randn(6, 16, 2, 8)  # [num_blocks, page 16, Hk 2, D 8]
    kw = {"k_cache": nhd, "v_cache": nhd, "block_table": torch.zeros(4000, 5, dtype=torch.int32),
          "cache_seqlens": torch.zeros(4000, dtype=torch.int32)}
    fix_paged_decode(kw, generator=g, page_dim=1)
    sl, bt = kw["cache_seqlens"], kw["block_table"]
    assert int(sl.min()) == 1 and int(sl.max()) == 5 * 16
    assert set(bt.unique().tolist()) == set(range(6))
    assert "max_seq_len" not in kw
    kw = {"k_cache": nhd, "v_cache": nhd, "block_table": torch.zeros(4000, 5, dtype=torch.int32),
          "cache_seqlens": torch.zeros(4000, dtype=torch.int32)}
    fix_paged_decode(kw, generator=g)  # reference geometry: page size = shape[-2] = 2
    assert int(kw["cache_seqlens"].max()) == 5 * 2
    with pytest.raises(ValueError):
        fix_paged_decode({"k_cache": nhd}, generator=g)


def test_compare_matched_ratio_boundary():
    """99% of elements matching passes; one element fewer fails."""
    ref = np.ones(1000, np.float32)
    out = ref.copy()
    out[:10] += 1.0  # 10 of 1000 outside -> matched 0.99
    st, max_abs, max_rel, matched, _ = oracle.compare(out, ref, "bf16")
    assert st == oracle.PASSED and matched == pytest.approx(0.99) and max_abs == 1.0
    assert max_rel == pytest.approx(1.0)
    out[10] += 1.0
    st, _, _, matched, detail = oracle.compare(out, ref, "bf16")
    assert st == oracle.INCORRECT_NUMERICAL and matched == pytest.approx(0.989)
    assert "atol=0.01" in detail


@pytest.mark.parametrize("tag,atol,rtol", [("f32", 1e-5, 1e-3), ("bf16", 1e-2, 1e-2),
                                           ("f16", 1e-2, 1e-2), ("fp8", 0.125, 0.125)])
def test_compare_tolerance_by_dtype(tag, atol, rtol):
    """An error at the bound matches (the test is a strict >); twice the bound does not.
    The tolerance follows the reference tensor's dtype, not the output's."""
    ref = np.full(100, 2.0, np.float32)
    bound = np.float32(atol + rtol * 2.0)
    at = ref + np.float32(bound * 0.999)
    assert oracle.compare(at, ref, tag)[3] == 1.0
    over = ref.copy()
    over[:2] += 2 * bound
    assert oracle.compare(over, ref, tag)[3] == pytest.approx(0.98)
    assert oracle.compare(over, ref, tag)[0] == oracle.INCORRECT_NUMERICAL


def test_compare_rejections():
    ref = np.arange(1, 9, dtype=np.float32)
    nan = ref.copy()
    nan[3] = np.nan
    inf = ref.copy()
    inf[0] = np.inf
    assert oracle.compare(nan, ref, "f32")[4] == "NaN in output"
    assert oracle.compare(inf, ref, "f32")[4] == "Inf in output"
    assert oracle.compare(np.zeros_like(ref), ref, "f32")[4] == "output is all-zeros"
    assert oracle.compare(ref[:4], ref, "f32")[0] == oracle.INCORRECT_SHAPE
    assert oracle.compare((ref,), (ref, ref), "f32")[0] == oracle.INCORRECT_SHAPE
    assert oracle.compare(ref, ref, "f32", out_dtypes="bf16")[0] == oracle.INCORRECT_DTYPE
    assert oracle.compare(ref, ref, "f32", out_dtypes="bf16", check_dtype=False)[0] == \
        oracle.PASSED
    # a NaN in a single element fails even though 99% of the rest match
    big = np.ones(1000, np.float32)
    bad = big.copy()
    bad[0] = np.nan
    assert oracle.compare(bad, big, "bf16")[0] == oracle.INCORRECT_NUMERICAL


def test_compare_leaves_and_order():
    """Nested structures flatten in order (dict values, tuples, lists; non-arrays dropped);
    the first failing leaf decides; empty leaves pass; the worst matched ratio is kept."""
    a = np.ones(100, np.float32)
    b = a.copy()
    b[:1] += 1.0  # 0.99 matched: passes
    out = {"x": (a, None), "y": [b, np.zeros(0, np.float32)]}
    ref = {"x": (a, 3), "y": [a, np.zeros(0, np.float32)]}
    st, _, _, matched, _ = oracle.compare(out, ref, ["f32", "f32", "f32"])
    assert st == oracle.PASSED and matched == pytest.approx(0.99)
    assert oracle.compare(np.zeros(0, np.float32), np.zeros(0, np.float32), "f32")[0] == \
        oracle.PASSED
    c = a.copy()
    c[:5] = -1.0
    assert oracle.compare((c, a), (a, a), "f32")[0] == oracle.INCORRECT_NUMERICAL
