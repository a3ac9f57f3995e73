"""fk_paged_decode_noalloc (the entry point whose split-context workspace is a static
device array) against fk_paged_decode with a caller-owned workspace, through the C ABI.

Both run the same kernels on the same plan, so the outputs must be identical bit for
bit.  Two calls in a row, the second on a smaller batch, check that the static scratch
carries nothing from one call into the next; a plan larger than the scratch is
rejected with FK_ERR_WORKSPACE before any launch.
"""
from __future__ import annotations

import pytest
import torch

from fastkernels_amd import _native, ops, workloads

pytestmark = pytest.mark.gpu


def _args(case, out, num_splits=0):
    b, hq, d = case.q.shape
    nb, bs, hk, _ = case.k_cache.shape
    plan = ops.paged_decode_plan(b, hq, hk, d, case.max_seq_len, num_splits)
    kvd = (_native.FK_DTYPE_FP8_E4M3FN if case.k_cache.dtype == torch.float8_e4m3fn
           else _native.FK_DTYPE_BF16)
    p = ops._ptr
    head = (p(out), out.stride(0), p(case.q), case.q.stride(0), p(case.k_cache), p(case.v_cache),
            kvd, p(case.k_scale), p(case.v_scale), p(case.block_tables),
            case.block_tables.stride(0), p(case.ctx_lens), b, hq, hk, d, bs, nb,
            float(case.scale), -1, p(None), plan.part_tokens, plan.max_parts)
    return head, plan


def _with_workspace(case, num_splits=0):
    out = torch.full_like(case.q, float("nan"))
    head, plan = _args(case, out, num_splits)
    ws = torch.zeros(max(1, plan.workspace_bytes), dtype=torch.uint8, device=case.q.device)
    _native.call("fk_paged_decode", *head, ops._ptr(ws), plan.workspace_bytes,
                 ops._stream(case.q))
    torch.cuda.synchronize()
    return out, plan


def _device_free_bytes() -> int:
    """Free device memory as hipMemGetInfo reports it (torch.cuda.mem_get_info calls
    it): unlike torch's allocator counters, it sees a hipMalloc made inside the library."""
    torch.cuda.synchronize()
    return torch.cuda.mem_get_info()[0]


_CALLED = False  # fk_paged_decode_noalloc already called in this process


def _noalloc(case, num_splits=0):
    """One fk_paged_decode_noalloc call.  Except on the process's first call (which may
    load the library's code object and with it the static scratch), device free memory
    must not drop across the call."""
    global _CALLED
    first, _CALLED = not _CALLED, True
    out = torch.full_like(case.q, float("nan"))
    head, _ = _args(case, out, num_splits)
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    free_before = _device_free_bytes()
    _native.call("fk_paged_decode_noalloc", *head, ops._stream(case.q))
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == before
    # The static scratch is part of the code object, loaded with the module: after the
    # first call nothing the library does may take device memory.
    if not first:
        assert _device_free_bytes() >= free_before
    return out


@pytest.mark.parametrize("num_splits", [0, 16])
def test_noalloc_matches_workspace_entry_point_twice(cuda, num_splits):
    """C3 at full size, then a smaller batch: bit-identical to fk_paged_decode both times."""
    print(f"noalloc: C3 then small batch, num_splits={num_splits}", flush=True)
    big = workloads.c3_decode(cuda, seed=200)
    ref_big, plan = _with_workspace(big, num_splits)
    assert plan.workspace_bytes <= 64 << 20  # FK_PAGED_DECODE_NOALLOC_MAX_BYTES
    _noalloc(big, num_splits)  # warm-up (the first call loads the scratch)
    got_big = _noalloc(big, num_splits)
    assert torch.equal(got_big, ref_big)
    small = workloads.c3_decode(cuda, batch=5, num_heads=16, kv_heads=4, pool_blocks=128,
                                ctx_lo=1, ctx_hi=3000, seed=7)
    ref_small, _ = _with_workspace(small, num_splits)
    got_small = _noalloc(small, num_splits)
    assert torch.equal(got_small, ref_small)


def test_noalloc_fp8_and_rejects_oversized_plan(cuda):
    """fp8 KV (C5 shape, two sequences) matches; a plan needing more workspace than the
    static scratch holds is refused with FK_ERR_WORKSPACE."""
    print("noalloc: fp8 and oversized plan", flush=True)
    case = workloads.c5_fp8_decode(cuda, batch=2, ctx_lens=[40000, 9000], seed=5)
    ref, _ = _with_workspace(case)
    assert torch.equal(_noalloc(case), ref)
    out = torch.empty_like(case.q)
    head, _ = _args(case, out)
    # fixed partitions over a huge max_seq_len: batch * heads * partitions rows of 512 B
    head = head[:-2] + (64, 60000)
    rc = _native.lib().fk_paged_decode_noalloc(*head, ops._stream(case.q))
    assert rc == _native.FK_ERR_WORKSPACE, rc
    assert "static scratch" in _native.lib().fk_last_error().decode()


_CAPTURE_FIRST_CALL = r"""
import sys
sys.path.insert(0, sys.argv[1])
import torch
from fastkernels_amd import _native, ops, workloads
import tests.test_zz_no_alloc as t

dev = torch.device("cuda:0")
case = workloads.c3_decode(dev, batch=9, num_heads=32, kv_heads=8, pool_blocks=256,
                           ctx_lo=1, ctx_hi=6000, seed=77)
ref, _ = t._with_workspace(case)
out = torch.full_like(case.q, float("nan"))
head, _ = t._args(case, out)
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    # The process's first fk_paged_decode_noalloc call: the scratch address is
    # resolved (hipGetSymbolAddress) while the stream is being captured.
    rc = _native.lib().fk_paged_decode_noalloc(*head, ops._stream(case.q))
assert rc == 0, (rc, _native.lib().fk_last_error())
for i in range(3):
    out.fill_(float("nan"))
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, ref), f"replay {i}"
print("capture-first-call OK", flush=True)
"""


def test_noalloc_first_call_inside_graph_capture(cuda, tmp_path):
    """A fresh process whose first fk_paged_decode_noalloc call is made under HIP graph
    capture: the capture succeeds, and every replay equals fk_paged_decode bit for bit."""
    import subprocess
    import sys
    from pathlib import Path

    print("noalloc: first call inside graph capture (fresh process)", flush=True)
    root = str(Path(__file__).resolve().parents[1])
    proc = subprocess.run([sys.executable, "-u", "-c", _CAPTURE_FIRST_CALL, root],
                          capture_output=True, text=True, timeout=100)
    assert proc.returncode == 0, proc.stdout[-2000:] + proc.stderr[-4000:]
    assert "capture-first-call OK" in proc.stdout
