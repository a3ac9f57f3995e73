"""GPU parity of the prefill's work-group key split (fk_paged_prefill_ws /
fk_varlen_prefill_ws): launches that would leave CUs without a work-group divide each
query block's keys over several work-groups, whose partial states a second kernel
merges.  Every case first checks that fk_prefill_split_plan asks for a workspace (so
the split is what runs), then compares against the oracle (atol = rtol = 1e-2 for bf16,
3e-2 for fp8 pages; log-sum-exp 1e-5), against the same call without the split, and
checks that a repeat is bit-identical."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from fastkernels_amd import _native, ops
from tests import test_gpu_prefill as P
from tests import test_gpu_prefill_heads as H

pytestmark = pytest.mark.gpu


def _flush(msg):
    print(msg, flush=True)


def _paged_ws_bytes(c, causal=True):
    fp8 = c["kc"].dtype == torch.float8_e4m3fn
    return _native.prefill_split_bytes(
        True, _native.FK_DTYPE_FP8_E4M3FN if fp8 else _native.FK_DTYPE_BF16,
        c["cu_q"].numel() - 1, c["q"].shape[0], c["max_q"], c["max_k"], c["q"].shape[1],
        c["kc"].shape[2], c["q"].shape[2], c["vc"].shape[3], causal)


def _plain(fn):
    """fn() with the library's launch without the work-group key split."""
    ops.PREFILL_SPLIT = False
    try:
        return fn()
    finally:
        ops.PREFILL_SPLIT = True


PAGED_CASES = [
    # (label, q_lens, k_lens, kwargs): each leaves CUs idle without the split
    ("chunk 256 over 4096, GQA 4", [256], [4096], {"hq": 8, "hk": 2, "bs": 256}),
    ("prompt 1024, MHA head 64 (paired blocks)", [1024], [1024],
     {"hq": 4, "hk": 4, "d": 64, "bs": 64}),
    ("chunks of a batch, one past its keys' parts", [1, 300, 50], [4000, 300, 2000],
     {"hq": 8, "hk": 2, "bs": 16}),
    ("fp8 pages", [256], [4096], {"hq": 8, "hk": 2, "bs": 64, "fp8": True}),
    ("head 256", [128, 7], [4096, 900], {"hq": 16, "hk": 2, "d": 256, "bs": 64}),
    ("GQA 8, head 64", [200], [3000], {"hq": 16, "hk": 2, "d": 64, "bs": 256}),
    # causal pairs at heads 128 and 256: the halves take the pair's blocks apart
    # (light block whole in the second half), each work-group on its part of both
    ("prompt 1024, GQA 4 head 128 (paired blocks)", [1024], [1024],
     {"hq": 8, "hk": 2, "bs": 64}),
    ("prompt 2048, head 256 (paired blocks)", [2048], [2048],
     {"hq": 8, "hk": 1, "d": 256, "bs": 64}),
    # 4-wave work-groups, two per CU, each block's keys in parts over work-groups
    # (in place of the 8-wave key split): chunks over cached keys at every head
    # size and page type, causal pairs at head 64
    ("prompt 2048, MHA head 64, 20 heads (4-wave work-groups)", [2048], [2048],
     {"hq": 20, "hk": 20, "d": 64, "bs": 256}),
    ("prompts 2x2048, MHA head 64, 10 heads (4-wave work-groups)", [2048, 2048], [2048, 2048],
     {"hq": 10, "hk": 10, "d": 64, "bs": 256}),
    ("chunks of 512 over 4000-8192 keys, GQA 4 (4-wave work-groups)", [512, 512, 300, 512],
     [8192, 6000, 8192, 4000], {"hq": 8, "hk": 2, "bs": 256}),
    ("fp8 pages, chunks over long caches (4-wave work-groups)", [512, 512, 300, 512],
     [8192, 6000, 8192, 4000], {"hq": 8, "hk": 2, "bs": 64, "fp8": True}),
    ("head 256, chunks of 512 over 8192 (4-wave work-groups)", [512] * 4, [8192] * 4,
     {"hq": 4, "hk": 1, "d": 256, "bs": 64}),
    ("chunks of a batch over long caches (4-wave work-groups)", [1, 300, 512],
     [8192, 5000, 4096], {"hq": 8, "hk": 2, "bs": 16}),
]


@pytest.mark.parametrize("label,q_lens,k_lens,kw", PAGED_CASES)
def test_paged_prefill_workgroup_key_split(cuda, label, q_lens, k_lens, kw):
    _flush(f"prefill work-group key split: {label}")
    c = P._case(cuda, q_lens, k_lens, seed=400 + len(label), **kw)
    assert _paged_ws_bytes(c) > 0, f"{label}: the launch does not split"
    tol = 3e-2 if kw.get("fp8") else 1e-2
    ref = P._oracle(c)
    got = P._run(c)
    P._close(got, ref, tol, f"{label}: split")
    P._close(_plain(lambda: P._run(c)), ref, tol, f"{label}: without the split")
    assert torch.equal(P._run(c), got), f"{label}: repeat differs"


# (q_lens, k_lens): the key split with parts, and (128 blocks over long caches) 4-wave
# work-groups with parts
_WINDOW_SHAPES = [([300, 9], [3000, 2500]), ([512, 300, 9, 512], [8192, 6000, 2500, 8192])]


@pytest.mark.parametrize("shape", [0, 1])
@pytest.mark.parametrize("window_left", [0, 100, 1000])
def test_paged_prefill_workgroup_key_split_window_and_sinks(cuda, window_left, shape):
    """A sliding window (parts whose stages all precede a query's window) and sinks,
    which join the sum once, in the merge."""
    _flush(f"prefill work-group key split window={window_left} shape={shape}")
    q_lens, k_lens = _WINDOW_SHAPES[shape]
    c = P._case(cuda, q_lens, k_lens, hq=8, hk=2, bs=16, seed=410 + window_left + shape)
    assert _paged_ws_bytes(c) > 0
    g = torch.Generator().manual_seed(411)
    sinks = (2 * torch.randn(8, generator=g)).float().to(cuda)
    ref = P._oracle(c, window_left=window_left, sinks=sinks)
    P._close(P._run(c, window_left=window_left, sinks=sinks), ref, 1e-2, "split")
    P._close(_plain(lambda: P._run(c, window_left=window_left, sinks=sinks)), ref, 1e-2,
             "without the split")


def test_paged_prefill_workgroup_key_split_noncausal(cuda):
    _flush("prefill work-group key split, causal=False")
    c = P._case(cuda, [64], [4096], hq=8, hk=2, bs=64, seed=420)
    assert _paged_ws_bytes(c, causal=False) > 0
    P._close(P._run(c, causal=False), P._oracle(c, causal=False), 1e-2, "non-causal split")


@pytest.mark.parametrize("hq,hk,d,dv,causal", [(8, 2, 128, 128, True), (4, 4, 64, 64, False),
                                               (2, 2, 192, 128, True), (8, 2, 80, 80, True)])
def test_varlen_prefill_workgroup_key_split_lse(cuda, hq, hk, d, dv, causal):
    """Dense keys with the log-sum-exp output (FlashAttnVarlen's return_softmax_lse):
    the merge forms it from the parts' fp32 sums; a causal chunk longer than its keys
    keeps rows with no visible key (lse -inf, output 0)."""
    _flush(f"varlen work-group key split {hq}/{hk}/{d}/{dv} causal={causal}")
    q_lens, k_lens = [600, 40], [2000, 20]
    q, k, v, cu_q, cu_k = H._dense(cuda, q_lens, k_lens, hq, hk, d, dv, seed=430 + d)
    nbytes = _native.prefill_split_bytes(False, _native.FK_DTYPE_BF16, 2, q.shape[0], 600, 2000,
                                         hq, hk, d, dv, causal)
    assert nbytes > 0
    scale = d ** -0.5
    ref_o, ref_l = H._oracle_dense(q, k, v, cu_q, cu_k, scale, causal, lse=True)
    out, lse = H._run_dense(q, k, v, cu_q, cu_k, 600, scale, causal, lse=True, max_k=2000)
    H._close(out, ref_o, 1e-2, "split output")
    H._lse_close(lse, ref_l, "split lse")
    out2, lse2 = _plain(lambda: H._run_dense(q, k, v, cu_q, cu_k, 600, scale, causal, lse=True,
                                             max_k=2000))
    H._close(out2, ref_o, 1e-2, "output without the split")
    H._lse_close(lse2, ref_l, "lse without the split")
    out3, lse3 = H._run_dense(q, k, v, cu_q, cu_k, 600, scale, causal, lse=True, max_k=2000)
    assert torch.equal(out3, out) and torch.equal(lse3, lse), "repeat differs"


@pytest.mark.parametrize("hq,hk,d,dv,causal,nseq", [(8, 2, 128, 128, True, 4),
                                                    (2, 2, 192, 128, False, 8),
                                                    (4, 4, 80, 80, False, 8)])
def test_varlen_prefill_key_parts_long_keys(cuda, hq, hk, d, dv, causal, nseq):
    """Dense keys, 512-query chunks over 8192 keys (128 blocks): 4-wave work-groups with
    each block's keys in parts over work-groups (in place of the 8-wave key split), with
    the log-sum-exp output."""
    _flush(f"varlen key parts over 8192 keys {hq}/{hk}/{d}/{dv} causal={causal} x{nseq}")
    q_lens, k_lens = [512] * nseq, [8192] * nseq
    q, k, v, cu_q, cu_k = H._dense(cuda, q_lens, k_lens, hq, hk, d, dv, seed=470 + d)
    nbytes = _native.prefill_split_bytes(False, _native.FK_DTYPE_BF16, nseq, q.shape[0], 512,
                                         8192, hq, hk, d, dv, causal)
    assert nbytes > 0
    scale = d ** -0.5
    ref_o, ref_l = H._oracle_dense(q, k, v, cu_q, cu_k, scale, causal, lse=True)
    out, lse = H._run_dense(q, k, v, cu_q, cu_k, 512, scale, causal, lse=True, max_k=8192)
    H._close(out, ref_o, 1e-2, "key parts output")
    H._lse_close(lse, ref_l, "key parts lse")
    out2, lse2 = _plain(lambda: H._run_dense(q, k, v, cu_q, cu_k, 512, scale, causal, lse=True,
                                             max_k=8192))
    H._close(out2, ref_o, 1e-2, "output without the parts")
    H._lse_close(lse2, ref_l, "lse without the parts")
    out3, lse3 = H._run_dense(q, k, v, cu_q, cu_k, 512, scale, causal, lse=True, max_k=8192)
    assert torch.equal(out3, out) and torch.equal(lse3, lse), "repeat differs"


def test_paged_prefill_ws_entry_point_contract(cuda):
    """fk_paged_prefill_ws: a NULL workspace runs the plain launch (bit-identical to
    fk_paged_prefill); one byte short of the plan is refused with FK_ERR_WORKSPACE
    before any launch; the planned size runs the split."""
    _flush("prefill ws entry point contract")
    c = P._case(cuda, [256], [4096], hq=8, hk=2, bs=256, seed=440)
    need = _paged_ws_bytes(c)
    assert need > 0
    lib = _native.lib()
    q = c["q"]
    batch = c["cu_q"].numel() - 1

    def call(ws, nbytes, entry="fk_paged_prefill_ws"):
        out = torch.full_like(q, float("nan"))
        args = [ops._ptr(out), out.stride(0), ops._ptr(q), q.stride(0), ops._ptr(c["kc"]),
                ops._ptr(c["vc"]), _native.FK_DTYPE_BF16, None, None, ops._ptr(c["bt"]),
                c["bt"].stride(0), ops._ptr(c["cu_q"]), ops._ptr(c["cu_k"]), batch, c["max_q"],
                c["max_k"], q.shape[1], c["kc"].shape[2], q.shape[2], q.shape[2],
                c["kc"].shape[1], c["kc"].shape[0], float(c["scale"]), 1, -1, None]
        if entry == "fk_paged_prefill_ws":
            args += [q.shape[0], ops._ptr(ws) if ws is not None else None, nbytes]
        rc = getattr(lib, entry)(*args, None)
        torch.cuda.synchronize()
        return rc, out

    rc_plain, plain = call(None, 0, "fk_paged_prefill")
    rc_null, null = call(None, 0)
    assert rc_plain == 0 and rc_null == 0
    assert torch.equal(null, plain), "NULL workspace differs from fk_paged_prefill"
    ws = torch.empty(need, dtype=torch.uint8, device=cuda)
    rc_short, _ = call(ws, need - 1)
    assert rc_short == _native.FK_ERR_WORKSPACE
    assert b"workspace" in lib.fk_last_error()
    rc_ok, split = call(ws, need)
    assert rc_ok == 0
    P._close(split, P._oracle(c), 1e-2, "ws entry point")


def test_prefill_split_plan_sizes():
    """The plan's workspace: parts x rows x heads x (value head size bf16 + 4 fp32),
    rounded up to 256 bytes; zero for launches that fill the GPU and for empty calls."""
    b = _native.prefill_split_bytes
    # a single 2048-token prompt over Qwen3-8B heads fills every CU: no split
    assert b(True, _native.FK_DTYPE_BF16, 1, 2048, 2048, 2048, 32, 8, 128, 128, True) == 0
    assert b(True, _native.FK_DTYPE_BF16, 1, 0, 0, 0, 32, 8, 128, 128, True) == 0
    nbytes = b(True, _native.FK_DTYPE_BF16, 1, 512, 512, 8192, 32, 8, 128, 128, True)
    rec = 512 * 32 * (128 * 2 + 4 * 4)
    assert nbytes > 0 and nbytes % 256 == 0 and nbytes % rec < 256
    parts = nbytes // rec
    assert 2 <= parts <= 8
    out = ctypes.c_int64(-1)
    assert _native.lib().fk_prefill_split_plan(1, 2, 1, 512, 512, 8192, 32, 7, 128, 128, 1,
                                               ctypes.byref(out)) == _native.FK_ERR_INVALID_ARG
    assert np.int64(out.value) == 0
