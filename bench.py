#!/usr/bin/env python3
"""Benchmark of the decode-step operator path on one MI355X.

Default workload (the headline metric): paged decode attention at the Qwen3-8B
shape, batch 64 (C3): q [64, 32, 128] bf16, 8 kv heads, 256-token pages from a
4096-block pool, context lengths ~ U[512, 8192].  One step = one
FlashAttnDecode-equivalent call (split-context partials kernel + merge kernel)
over the batch, with all inputs resident in HBM.

Prints ONE JSON line: value = whole-call throughput in algorithmic GB/s
(K+V bytes attended + q + out + block-table entries + ctx, per call, divided by
the mean step time of K back-to-back calls), the per-call time, the roofline of
the dominant kernel (the partials kernel, timed live with a HIP event pair on its
stream around each of max(10, K) calls run right after the timed ones: event
markers delay the next launch, so none sit among the timed calls) against the
8 TB/s HBM peak, the same call replayed from a HIP
graph, and the reference's PyTorch decode path (oracle/torch_path.py) timed over
the whole batch on the host's cores.

  python bench.py [--steps K] [--warmup W] [--num-splits S] [--no-cpu]
  python bench.py --table          # per-op table for C1-C5 to stderr (+ --table-json PATH)
  python bench.py --calib-copy     # plain 1 GiB device copy, for rocprof counter scaling
  python bench.py --profile-ops    # each op after a cache flush, for rocprof counter passes
  python bench.py --profile-prefill  # the table's prefill cases, for rocprof counter passes
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "paged decode attn µs/call + achieved HBM GB/s (% of 8 TB/s), Qwen3-8B bs64"


def _parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--num-splits", type=int, default=0, help="0 = automatic partitioning")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline time budget")
    ap.add_argument("--table", action="store_true", help="per-op table for C1-C5")
    ap.add_argument("--table-json", type=str, default=None)
    ap.add_argument("--calib-copy", action="store_true")
    ap.add_argument("--profile-ops", action="store_true",
                    help="each op on its C1-C5 inputs after a cache flush, for rocprofv3 --pmc")
    ap.add_argument("--profile-prefill", action="store_true",
                    help="the table's prefill cases after a cache flush, for rocprofv3")
    ap.add_argument("--seed", type=int, default=200)
    ap.add_argument("--block-size", type=int, default=256,
                    help="C3's page size in tokens (the pool keeps C3's 1 GiB per cache: "
                         "4096 * 256 / block_size pages)")
    return ap.parse_args()


def _flush_buffer(device):
    import torch

    # Twice the 256 MB MALL (Infinity Cache): reading it evicts L2 and MALL between
    # timed calls.  A read (not a fill) leaves no dirty lines whose write-back
    # would compete with the timed kernel.
    return torch.ones(512 * 1024 * 1024 // 4, dtype=torch.float32, device=device)


KERNEL_SAMPLES = 10  # bench_decode: HIP-event samples of the partials kernel per run (at least)


class HipEvents:
    """HIP events created with hipEventDisableSystemFence, recorded on a given stream.

    A default event (torch.cuda.Event) performs a system-scope release when it is
    recorded: on MI355X that writes back and invalidates the caches, which measured
    ~6 us per event pair on the C3 step (and slows the next kernel).  These timing
    events skip that fence (hip_runtime_api.h: "events that are only being used to
    measure timing"): ~2 us per pair, and they time the kernel within 1 us of the
    rocprofv3 trace."""

    FLAG_DISABLE_SYSTEM_FENCE = 0x20000000

    def __init__(self, n: int):
        import ctypes

        self._ct = ctypes
        hip = ctypes.CDLL("libamdhip64.so")
        hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                            ctypes.c_void_p]
        hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self._hip = hip
        self.ev = []
        for _ in range(n):
            e = ctypes.c_void_p()
            rc = hip.hipEventCreateWithFlags(ctypes.byref(e), self.FLAG_DISABLE_SYSTEM_FENCE)
            if rc != 0:
                raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")
            self.ev.append(e)

    def record(self, i: int, stream_handle: int) -> None:
        rc = self._hip.hipEventRecord(self.ev[i], self._ct.c_void_p(stream_handle))
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def elapsed_ms(self, i: int, j: int) -> float:
        f = self._ct.c_float()
        rc = self._hip.hipEventElapsedTime(self._ct.byref(f), self.ev[i], self.ev[j])
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return f.value

    def close(self) -> None:
        for e in self.ev:
            self._hip.hipEventDestroy(e)
        self.ev = []


def settle_clocks(fn, seconds=0.3):
    """Run fn back to back for `seconds` of wall time before anything is timed.

    An idle MI355X takes tens of milliseconds of sustained load to reach its steady
    clocks: measured on C5, the first ~25 calls of a process (~10 ms) ran up to 30%
    slower than the rest, whatever op came first.  A fixed number of warmup calls
    does not cover that for short ops, so the bench first loads the GPU for a fixed
    time (untimed), then does its warmup steps."""
    import torch

    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(20):
            fn()
        torch.cuda.synchronize()


def time_call(fn, iters=50, warmup=10, flush=None):
    """Median and mean of fn's GPU time (fence-free HIP events bracket only fn; an
    optional cache flush is enqueued before each start event)."""
    import torch

    for _ in range(warmup):
        fn()
    ev = HipEvents(2 * iters)
    sh = torch.cuda.current_stream().cuda_stream
    sink = None
    for i in range(iters):
        if flush is not None:
            sink = flush.sum()
        ev.record(2 * i, sh)
        fn()
        ev.record(2 * i + 1, sh)
    torch.cuda.synchronize()
    del sink
    ms = [ev.elapsed_ms(2 * i, 2 * i + 1) for i in range(iters)]
    ev.close()
    return statistics.median(ms), statistics.fmean(ms)


ROTATE_BYTES = 512 * 1024 * 1024  # twice the 256 MB MALL


def time_rotated(fns, iters=20, warmup=3):
    """µs per call of fns run back to back inside one captured HIP graph, median of
    `iters` replays.  Each fn works on its own inputs, and together they touch more
    than the MALL holds (ROTATE_BYTES), so every call reads its inputs from HBM, as
    after a flush; the graph removes the host's launch overhead and the per-call
    event pair, which dominate a single timed call of a few-µs kernel.  This is the
    setting of a graph-replayed engine step (engine.py:5386-5428)."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for fn in fns:
            fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for fn in fns:
            fn()
    for _ in range(warmup):
        graph.replay()
    ev = HipEvents(2 * iters)
    sh = torch.cuda.current_stream().cuda_stream
    for i in range(iters):
        ev.record(2 * i, sh)
        graph.replay()
        ev.record(2 * i + 1, sh)
    torch.cuda.synchronize()
    ms = statistics.median(ev.elapsed_ms(2 * i, 2 * i + 1) for i in range(iters))
    ev.close()
    del graph
    return ms * 1e3 / len(fns)


def copies_for(footprint: int) -> int:
    """Input sets needed so that one pass over them touches ROTATE_BYTES."""
    return max(2, -(-ROTATE_BYTES // max(1, footprint)))


# ---------------------------------------------------------------------------
# CPU baseline: the reference's PyTorch decode path (Attention._decode_torch,
# attention_impl.py:592-664), restated in oracle/torch_path.py, on the host cores
# ---------------------------------------------------------------------------
def cpu_baseline_decode(case, budget_s: float, gpu_out=None):
    """Times oracle.torch_path.decode_torch (per-sequence page gather, repeat_interleave,
    F.scaled_dot_product_attention, bf16) over the WHOLE C3 batch on the host, with
    torch's intra-op threads set to every core this process may use.  Only the pages
    the batch uses are copied to the host (the block tables are renumbered to match),
    which changes no value the path reads."""
    import torch

    from oracle.torch_path import decode_torch

    cores_avail = len(os.sched_getaffinity(0))
    # The GPU box sets OMP_NUM_THREADS to this process's CPU share; use all of it.
    threads = min(cores_avail, int(os.environ.get("OMP_NUM_THREADS", cores_avail) or cores_avail))
    prev_threads = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        bs = case.k_cache.shape[1]
        ctx = case.ctx_lens.to(torch.int64)
        pages = (ctx + bs - 1) // bs
        bt = case.block_tables.to(torch.int64)
        used = torch.cat([bt[i, :int(pages[i])] for i in range(bt.shape[0])])
        k_host = case.k_cache[used].cpu()
        v_host = case.v_cache[used].cpu()
        # sequence i's pages are rows [off_i, off_i + pages_i) of the compacted caches
        off = torch.cumsum(pages, 0) - pages
        bt_host = torch.full(tuple(bt.shape), -1, dtype=torch.int32)
        for i in range(bt.shape[0]):
            bt_host[i, :int(pages[i])] = torch.arange(int(off[i]), int(off[i] + pages[i]),
                                                      dtype=torch.int32)
        q_host = case.q.cpu()
        ctx_host = case.ctx_lens.cpu()
        out = decode_torch(q_host, k_host, v_host, ctx_host, bt_host, case.scale)  # warmup
        times = []
        t_end = time.perf_counter() + budget_s
        while not times or time.perf_counter() < t_end:
            t0 = time.perf_counter()
            out = decode_torch(q_host, k_host, v_host, ctx_host, bt_host, case.scale)
            times.append(time.perf_counter() - t0)
    finally:
        torch.set_num_threads(prev_threads)
    el = statistics.median(times)
    total_bytes = case.algorithmic_bytes()
    res = {
        "value": round(total_bytes / el / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle.torch_path.decode_torch (the reference's _decode_torch, "
                   f"attention_impl.py:592-664: page gather, repeat_interleave, "
                   f"F.scaled_dot_product_attention in bf16) over the whole C3 batch "
                   f"({case.q.shape[0]} sequences, {int(ctx.sum())} cached tokens), "
                   f"median of {len(times)} calls in {budget_s:.0f}s; "
                   f"torch threads {threads} of {cores_avail} cores in this process's "
                   f"affinity mask"),
        "us_per_call": round(el * 1e6, 1),
        "torch_threads": threads,
        "cores_in_affinity": cores_avail,
    }
    if gpu_out is not None:  # the two outputs side by side (a sanity check, not the parity test)
        diff = (out.float() - gpu_out.float().cpu()).abs()
        res["max_abs_vs_gpu"] = float(f"{diff.max().item():.3g}")
    return res


# ---------------------------------------------------------------------------
# Headline: paged decode C3
# ---------------------------------------------------------------------------
def bench_decode(args):
    import torch

    from fastkernels_amd import ops, workloads

    dev = torch.device("cuda:0")
    case = workloads.c3_decode(dev, seed=args.seed, block_size=args.block_size,
                               pool_blocks=4096 * 256 // args.block_size)
    b, hq, d = case.q.shape
    hk = case.k_cache.shape[2]
    part, nparts, wsb = ops.paged_decode_plan(b, hq, hk, d, case.max_seq_len, args.num_splits)
    ws = torch.zeros(max(1, wsb),
                     dtype=torch.uint8, device=dev)
    out = torch.empty_like(case.q)
    partials, reduce = ops.paged_decode_phases(out, case.q, case.k_cache, case.v_cache,
                                               case.block_tables, case.ctx_lens, case.scale,
                                               part, nparts, ws)
    total_bytes = case.algorithmic_bytes()
    out_bytes = out.numel() * out.element_size()
    partial_bytes = total_bytes - out_bytes  # the main kernel's algorithmic bytes (no output)
    def step():
        partials()
        reduce()

    settle_clocks(step)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream
    # Timed pass (`value`): K back-to-back calls and nothing else on the stream.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        partials()
        reduce()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    # Event pass (`roofline.achieved`): the same K calls again, each partials launch
    # between a pair of HIP events recorded on its stream (without the system-scope
    # fence).  An event marker holds the next launch back by a few µs, so the
    # markers stay out of the timed pass; its wall clock is reported beside.
    nsamp = max(KERNEL_SAMPLES, args.steps)
    ev = HipEvents(2 * nsamp)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for j in range(nsamp):
        ev.record(2 * j, sh)
        partials()
        ev.record(2 * j + 1, sh)
        reduce()
    torch.cuda.synchronize()
    ev_pass_us = (time.perf_counter() - t1) * 1e6 / nsamp
    kern_ms = [ev.elapsed_ms(2 * k, 2 * k + 1) for k in range(nsamp)]
    ev.close()
    kavg = statistics.fmean(kern_ms)
    achieved = partial_bytes / (kavg * 1e-3) / 1e9
    graph_us = _graph_replay_us(lambda: ops.paged_decode(
        out, case.q, case.k_cache, case.v_cache, case.block_tables, case.ctx_lens, case.scale,
        part, nparts, ws), replays=max(20, args.steps))
    step_calls, step_us, step_eager_us = _graph_step_us(case, part, nparts, ws, args.seed)
    result = {
        "metric": METRIC,
        "value": round(total_bytes / (ms_per_step * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "us_per_call": round(ms_per_step * 1e3, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/KV, ctx ~ U[512,8192], random-permutation block tables)",
        "config": {
            "workload": "C3 paged decode attention, Qwen3-8B shape, batch 64",
            "batch": b, "num_heads": hq, "num_kv_heads": hk, "head_dim": d,
            "block_size": case.k_cache.shape[1], "pool_blocks": case.k_cache.shape[0],
            "sum_ctx": int(case.ctx_lens.to(torch.int64).sum().item()),
            "part_tokens": part, "max_parts": nparts, "seed": args.seed,
            "algorithmic_bytes_per_call": total_bytes,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "paged_decode_balanced_kernel" if part == 0 else "paged_decode_partition_kernel",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": _committed_traffic(
                "paged_decode_balanced_kernel" if part == 0 else "paged_decode_partition_kernel",
                part, case.k_cache.shape[1]) if args.seed == 200 else None,
            "traffic_source": "profiles/paged_decode_c3_traffic.json (rocprofv3 FETCH_SIZE/WRITE_SIZE, copy-calibrated)",
            "avg_kernel_us": round(kavg * 1e3, 2),
            "kernel_samples": len(kern_ms),
            "kernel_events": ("an event pair around every partials launch of an event pass "
                              "of max(10, steps) calls run right after the timed pass"),
            "event_pass_us_per_call": round(ev_pass_us, 2),
            "algorithmic_bytes_per_launch": partial_bytes,
        },
        # The same call as the engine's decode step runs it: both launches captured
        # in one HIP graph and replayed (engine.py:5386-5428).  Reported beside the
        # eager figure above, which is `value`.
        "graph_replay": {"us_per_call": round(graph_us, 2),
                         "GBs": round(total_bytes / (graph_us * 1e-6) / 1e9, 1),
                         "frac": round(total_bytes / (graph_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)},
        # The engine captures a whole decode step -- every layer's attention -- in one
        # graph (engine.py:5386-5428): Qwen3-8B's 36 layers' decode calls, each on its
        # own q / out and on one of four cache sets in turn (so no call finds its
        # predecessor's pages in the MALL), replayed; µs per call = replay / 36
        # (median of 10 replays).  `eager_us_per_call`: the same 36 calls launched
        # eagerly, timed in alternation with the replays.
        "graph_step": {"calls": step_calls, "us_per_call": round(step_us, 2),
                       "GBs": round(total_bytes / (step_us * 1e-6) / 1e9, 1),
                       "frac": round(total_bytes / (step_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                       "eager_us_per_call": round(step_eager_us, 2),
                       "eager_frac": round(total_bytes / (step_eager_us * 1e-6) / 1e9
                                           / HBM_PEAK_GBS, 4)},
    }
    return result, case, out


def _graph_replay_us(call, replays: int) -> float:
    """Wall-clock µs per replay of `call` captured alone in a HIP graph, over `replays`
    back-to-back replays (after 3 untimed ones)."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(replays):
        graph.replay()
    torch.cuda.synchronize()
    us = (time.perf_counter() - t0) * 1e6 / replays
    del graph
    return us


def _graph_step_us(case, part: int, nparts: int, ws, seed: int, layers: int = 36,
                   cache_sets: int = 4, replays: int = 10) -> tuple[int, float, float]:
    """µs per decode call when `layers` calls (a decode step of Qwen3-8B's 36 layers) are
    captured in one HIP graph and replayed: each call has its own q and out, and the
    calls cycle over `cache_sets` K/V cache pairs of C3's shape (the first is C3's own;
    the others hold other seeded values), with C3's block tables and lengths.  One
    workspace serves the calls, which run one after another on the stream.  Returns
    (calls, graph µs per call, eager µs per call)."""
    import torch

    from fastkernels_amd import ops

    dev = case.q.device
    caches = [(case.k_cache, case.v_cache)]
    for i in range(1, cache_sets):
        g = torch.Generator(device=dev)
        g.manual_seed(seed + 1000 + i)
        kc = torch.randn(case.k_cache.shape, generator=g, device=dev,
                         dtype=torch.float32).to(torch.bfloat16)
        vc = torch.randn(case.k_cache.shape, generator=g, device=dev,
                         dtype=torch.float32).to(torch.bfloat16)
        caches.append((kc, vc))
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 2000)
    qs = [torch.randn(case.q.shape, generator=g, device=dev).to(torch.bfloat16)
          for _ in range(layers)]
    outs = [torch.empty_like(case.q) for _ in range(layers)]

    def step():
        for i in range(layers):
            kc, vc = caches[i % cache_sets]
            ops.paged_decode(outs[i], qs[i], kc, vc, case.block_tables, case.ctx_lens,
                             case.scale, part, nparts, ws)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    # Untimed load first, as before the headline (settle_clocks): the cache sets were
    # just written, and the first few hundred calls on freshly written pools run a
    # few percent slower than the steady state an engine decodes in.
    settle_clocks(graph.replay, seconds=0.3)
    torch.cuda.synchronize()
    # The replays alternate with the same 36 calls launched eagerly, so that the
    # two figures see the same clocks (a sustained load runs a few percent slower
    # than the first second after idle; measuring one after the other would put
    # that difference between them).
    g_us, e_us = [], []
    for _ in range(replays):
        t0 = time.perf_counter()
        graph.replay()
        torch.cuda.synchronize()
        g_us.append((time.perf_counter() - t0) * 1e6 / layers)
        t0 = time.perf_counter()
        step()
        torch.cuda.synchronize()
        e_us.append((time.perf_counter() - t0) * 1e6 / layers)
    del graph, caches, qs, outs
    torch.cuda.empty_cache()
    return layers, statistics.median(g_us), statistics.median(e_us)


def _committed_traffic(kernel: str, part: int, block_size: int = 256):
    """HBM bytes per launch of the dominant kernel from the committed rocprof PMC
    summary (profiles/paged_decode_c3_traffic.json), if it covers this kernel and page
    size."""
    path = ROOT / "profiles" / "paged_decode_c3_traffic.json"
    try:
        d = json.loads(path.read_text())
    except (OSError, ValueError):
        return None
    if (d.get("workload") != "C3" or d.get("part_tokens") != part
            or kernel not in d.get("kernel", "") or d.get("block_size", 256) != block_size):
        return None
    return d.get("traffic_bytes")


def _cpu_time(fn, budget_s: float = 2.0) -> tuple[float, int]:
    """Median seconds of fn over as many runs as fit in budget_s (after one warmup)."""
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while not times or time.perf_counter() < t_end:
        t0 = time.perf_counter_ns()
        fn()
        times.append((time.perf_counter_ns() - t0) * 1e-9)
    return statistics.median(times), len(times)


def _np(t):
    return t.detach().float().cpu().numpy()


def bench_table(args):
    """Per-op µs/call and GB/s for C1-C5 on the GPU (L2 + MALL flushed before each
    timed call), each beside the reference's PyTorch path for the op (restated in
    oracle/torch_path.py) timed on this host's cores, and a parity verdict against
    the numpy oracle."""
    import numpy as np
    import torch

    import oracle
    from fastkernels_amd import ops, workloads

    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        threadpool_limits = None
    cores = min(len(os.sched_getaffinity(0)), 16)
    limiter = threadpool_limits(limits=cores) if threadpool_limits else None
    torch.set_num_threads(cores)
    dev = torch.device("cuda:0")
    flush = _flush_buffer(dev)
    rows = []
    settle_clocks(lambda: flush.sum())

    def verdict(out, ref, tags, bitexact=None):
        """The reference bench's acceptance status of out against the oracle's ref
        (oracle.compare: 99% of elements within the dtype's atol/rtol)."""
        st, max_abs, max_rel, matched, _ = oracle.compare(out, ref, tags)
        v = {"status": st, "max_abs": float(f"{max_abs:.3g}"), "max_rel": float(f"{max_rel:.3g}"),
             "matched": round(matched, 5)}
        if bitexact is not None:
            v["bitexact"] = bool(bitexact)
        return v

    def add(cfg, op, fn, nbytes, cpu=None, iters=50, parity=None, rotated=None):
        """cpu = (callable, fraction of the op's bytes it processes, sample text) or None;
        parity = a callable giving verdict(...) for one call on fresh inputs, or None;
        rotated = a callable giving the per-input-set calls for time_rotated, or None
        (run last: it may write the op's outputs many times over)."""
        med, mean = time_call(fn, iters=iters, warmup=5, flush=flush)
        row = {"config": cfg, "op": op, "us_median": round(med * 1e3, 2),
               "us_mean": round(mean * 1e3, 2), "bytes": nbytes,
               "GBs": round(nbytes / (med * 1e-3) / 1e9, 1),
               "frac_of_8TBs": round(nbytes / (med * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        if cpu is not None:
            cfn, frac, sample = cpu
            sec, reps = _cpu_time(cfn)
            row["cpu"] = {"us_per_call": round(sec / frac * 1e6, 1),
                          "GBs": round(nbytes * frac / sec / 1e9, 3), "cores": cores,
                          "kind": "port", "sample": f"{sample}; median of {reps}"}
        if parity is not None:
            row["parity"] = parity()
        if rotated is not None:
            fns = rotated()
            us = time_rotated(fns)
            row["graph"] = {"us_per_call": round(us, 2), "copies": len(fns),
                            "GBs": round(nbytes / (us * 1e-6) / 1e9, 1),
                            "frac_of_8TBs": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
            del fns
            torch.cuda.empty_cache()
        rows.append(row)
        print(json.dumps(row), file=sys.stderr, flush=True)

    # C1: fused add+RMSNorm; CPU path in fp32 (forward_native), GPU in bf16.
    c1 = workloads.c1_norm(dev)
    from oracle import torch_path as tp

    c1f = workloads.c1_norm("cpu", dtype=torch.float32)
    x, r = c1.x.clone(), c1.residual.clone()
    def norm_copies(x0, r0, w):
        sets = [(x0.clone(), r0.clone()) for _ in range(copies_for(4 * x0.numel() * 2))]
        return [lambda xx=xx, rx=rx: ops.fused_add_rms_norm(xx, rx, w, 1e-6) for xx, rx in sets]

    def norm_parity(case):
        xx, rx = case.x.clone() if hasattr(case, "x") else case.hidden.clone(), case.residual.clone()
        w = case.weight if hasattr(case, "weight") else case.norm_weight
        x0, r0 = _np(xx), _np(rx)
        ops.fused_add_rms_norm(xx, rx, w, 1e-6)
        ref = oracle.rms_norm(x0, _np(w), 1e-6, "bf16", residual=r0)
        return verdict((_np(xx), _np(rx)), ref, "bf16")

    add("C1", "fused_add_rmsnorm bf16 [256,1024]",
        lambda: ops.fused_add_rms_norm(x, r, c1.weight, c1.eps), (4 * 256 * 1024 + 1024) * 2,
        (lambda: tp.rms_norm_native(c1f.x, c1f.weight, 1e-6, residual=c1f.residual), 2.0,
         "torch RMSNorm.forward_native (rms_norm.py:97-118) fp32 on the full [256,1024] "
         "(4,198,400 B; GB/s on the fp32 bytes)"),
        parity=lambda: norm_parity(c1), rotated=lambda: norm_copies(c1.x, c1.residual, c1.weight))
    # C2: store_kvcache (bit copy); CPU: in-place numpy scatter into full-size caches.
    c2 = workloads.c2_store(dev)
    nvalid = int((c2.slot_mapping >= 0).sum().item())

    def store_copies(key, value, kc, vc, valid_frac):
        """Input sets of fresh rows and slots (a new draw of distinct slots per set, the
        same share of -1) into the given caches."""
        n = key.shape[0]
        row = key[0].numel() * key.element_size()
        g = torch.Generator().manual_seed(workloads.SEED + 99)
        sets = []
        for _ in range(copies_for(n * row * 4)):
            sl = torch.randperm(kc.shape[0] * kc.shape[1], generator=g)[:n]
            sl[torch.rand(n, generator=g) >= valid_frac] = -1
            sets.append((torch.randn(key.shape, generator=g).to(key.dtype).to(dev),
                         torch.randn(key.shape, generator=g).to(key.dtype).to(dev), sl.to(dev)))
        return [lambda k_=k_, v_=v_, s_=s_: ops.store_kvcache(k_, v_, kc, vc, s_)
                for k_, v_, s_ in sets]

    def store_parity(kc, vc, ek, ev):
        """Whole caches against the oracle's (which the CPU leg has just filled)."""
        gk, gv = kc.view(torch.int16).cpu().numpy(), vc.view(torch.int16).cpu().numpy()
        exact = np.array_equal(gk, ek) and np.array_equal(gv, ev)
        bf = lambda a: oracle.bf16_bits_to_f32(a.view(np.uint16).reshape(-1))
        return verdict((bf(gk), bf(gv)), (bf(ek), bf(ev)), "bf16", bitexact=exact)

    k2 = c2.key.view(torch.int16).cpu().numpy()
    v2 = c2.value.view(torch.int16).cpu().numpy()
    s2 = c2.slot_mapping.cpu().numpy()
    kc2 = np.zeros(tuple(c2.k_cache.shape), np.int16)
    vc2 = np.zeros_like(kc2)
    oracle.store_kvcache_(k2, v2, kc2, vc2, s2)  # the parity reference
    kt2, vt2, st2 = c2.key.cpu(), c2.value.cpu(), c2.slot_mapping.cpu()
    kct2 = torch.zeros(tuple(c2.k_cache.shape), dtype=torch.bfloat16)
    vct2 = torch.zeros_like(kct2)
    add("C2", "store_kvcache [4096,8,128]",
        lambda: ops.store_kvcache(c2.key, c2.value, c2.k_cache, c2.v_cache, c2.slot_mapping),
        8 * 4096 + nvalid * 4 * 8 * 128 * 2,
        (lambda: tp.store_kvcache_torch(kt2, vt2, kct2, vct2, st2), 1.0,
         "torch index_copy_ scatter of the C2 rows into full-size host caches"),
        parity=lambda: store_parity(c2.k_cache, c2.v_cache, kc2, vc2),
        rotated=lambda: store_copies(c2.key, c2.value, c2.k_cache, c2.v_cache, nvalid / 4096))
    del c2, kc2, vc2, kct2, vct2
    # C4 chain ops
    c4 = workloads.c4_chain(dev)
    h, rr = c4.hidden.clone(), c4.residual.clone()
    hc4, rc4, wc4 = c4.hidden.cpu(), c4.residual.cpu(), c4.norm_weight.cpu()
    add("C4", "fused_add_rmsnorm bf16 [256,4096]",
        lambda: ops.fused_add_rms_norm(h, rr, c4.norm_weight, 1e-6), (4 * 256 * 4096 + 4096) * 2,
        (lambda: tp.rms_norm_native(hc4, wc4, 1e-6, residual=rc4), 1.0,
         "torch RMSNorm.forward_native bf16 on the full [256,4096]"),
        parity=lambda: norm_parity(c4),
        rotated=lambda: norm_copies(c4.hidden, c4.residual, c4.norm_weight))
    from fastkernels_amd.candidate.L1.rotary_emb import RotaryEmbedding

    rope = RotaryEmbedding(128, c4.max_position, c4.rope_theta).to(dev)
    qkv = c4.qkv.clone()
    q, k = qkv[:, :4096], qkv[:, 4096:5120]
    pn, csn = c4.positions.cpu().numpy(), _np(rope.cos_sin_cache)
    qt4, kt4, pt4, cst4 = q.cpu(), k.cpu(), c4.positions.cpu(), rope.cos_sin_cache.cpu()

    def rope_copies():
        sets = [c4.qkv.clone() for _ in range(copies_for(2 * 256 * 5120 * 2))]
        return [lambda t=t: ops.rotary_embedding(c4.positions, t[:, :4096], t[:, 4096:5120], 128,
                                                 rope.cos_sin_cache, True) for t in sets]

    def rope_parity():
        qkv_p = c4.qkv.clone()
        qp, kp = qkv_p[:, :4096], qkv_p[:, 4096:5120]
        ref = oracle.rotary(pn, _np(qp), _np(kp), 128, csn, True, "bf16")
        ops.rotary_embedding(c4.positions, qp, kp, 128, rope.cos_sin_cache, True)
        return verdict((_np(qp), _np(kp)), ref, "bf16")

    add("C4", "rotary q[256,32x128] k[256,8x128]",
        lambda: ops.rotary_embedding(c4.positions, q, k, 128, rope.cos_sin_cache, True),
        2 * 256 * 5120 * 2 + 256 * 8 + 256 * 128 * 4,
        (lambda: tp.rotary_native(pt4, qt4, kt4, 128, cst4), 1.0,
         "torch RotaryEmbedding.forward_native (NeoX) on the full q/k"), parity=rope_parity,
        rotated=rope_copies)
    v = qkv[:, 5120:]
    dec = c4.decode
    # Qwen3 attention prologue at C4: per-head q/k RMSNorm + rotary + store_kvcache,
    # as the separate ops (norm of each head row, then rotary, then store) and fused.
    g = torch.Generator().manual_seed(workloads.SEED + 7)
    qw = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16).to(dev)
    kw = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16).to(dev)
    qkv_a = c4.qkv.clone()
    qa, ka, va = qkv_a[:, :4096], qkv_a[:, 4096:5120], qkv_a[:, 5120:]
    qrows = torch.empty(256, 32, 128, dtype=torch.bfloat16, device=dev)
    krows = torch.empty(256, 8, 128, dtype=torch.bfloat16, device=dev)

    def qk_separate():
        ops.rms_norm(qrows, qa.view(256, 32, 128).contiguous(), qw, 1e-6)
        ops.rms_norm(krows, ka.view(256, 8, 128).contiguous(), kw, 1e-6)
        qa.copy_(qrows.view(256, 4096))
        ka.copy_(krows.view(256, 1024))
        ops.rotary_embedding(c4.positions, qa, ka, 128, rope.cos_sin_cache, True)
        ops.store_kvcache(ka.view(256, 8, 128), va.view(256, 8, 128), dec.k_cache, dec.v_cache,
                          c4.slot_mapping)

    def qk_fused():
        ops.qk_norm_rope_store(c4.positions, qa, ka, va, dec.k_cache, dec.v_cache,
                               c4.slot_mapping, 128, rope.cos_sin_cache, True, qw, kw, 1e-6)

    qk_bytes = (256 * (4096 + 2 * 1024) * 2 + 256 * (4096 + 1024) * 2 + 256 * 2 * 1024 * 2
                + 256 * 16 + 256 * 128 * 4 + 2 * 128 * 2)
    add("C4", "q/k RMSNorm + rotary + store_kvcache, separate (the reference's op sequence)",
        qk_separate, qk_bytes)
    def qk_fused_copies():
        """Input sets for the fused prologue: fresh qkv rows and slots into scratch caches
        (the decode case's cache keeps its contents)."""
        gs = torch.Generator().manual_seed(workloads.SEED + 98)
        kcs = torch.zeros(1024, 256, 8, 128, dtype=torch.bfloat16, device=dev)
        vcs = torch.zeros_like(kcs)
        sets = [(c4.qkv.clone(), torch.randperm(1024 * 256, generator=gs)[:256].to(dev))
                for _ in range(copies_for(qk_bytes))]
        return [lambda t=t, sl=sl: ops.qk_norm_rope_store(
            c4.positions, t[:, :4096], t[:, 4096:5120], t[:, 5120:], kcs, vcs, sl, 128,
            rope.cos_sin_cache, True, qw, kw, 1e-6) for t, sl in sets]

    add("C4", "q/k RMSNorm + rotary + store_kvcache, fused (qk_norm_rope_store)", qk_fused,
        qk_bytes, rotated=qk_fused_copies)
    kt16, vt16 = k.contiguous().view(256, 8, 128).cpu(), v.contiguous().view(256, 8, 128).cpu()
    st4 = c4.slot_mapping.cpu()

    # scratch caches for the rotated C4 store (the decode case's caches stay as they are)
    scratch_kc = torch.zeros(1024, 256, 8, 128, dtype=torch.bfloat16, device=dev)
    scratch_vc = torch.zeros_like(scratch_kc)

    def store_rows_parity():
        """The cache rows at the C4 slots against the stored key/value rows."""
        kc_ = dec.k_cache.view(-1, 8 * 128)[c4.slot_mapping].view(torch.int16).cpu().numpy()
        vc_ = dec.v_cache.view(-1, 8 * 128)[c4.slot_mapping].view(torch.int16).cpu().numpy()
        ek = k.contiguous().view(torch.int16).reshape(256, -1).cpu().numpy()
        ev = v.contiguous().view(torch.int16).reshape(256, -1).cpu().numpy()
        exact = np.array_equal(kc_, ek) and np.array_equal(vc_, ev)
        bf = lambda a: oracle.bf16_bits_to_f32(a.view(np.uint16))
        return verdict((bf(kc_), bf(vc_)), (bf(ek), bf(ev)), "bf16", bitexact=exact)
    cache_t = torch.zeros(tuple(dec.k_cache.shape), dtype=torch.bfloat16)
    add("C4", "store_kvcache [256,8,128]",
        lambda: ops.store_kvcache(k.view(256, 8, 128), v.view(256, 8, 128), dec.k_cache,
                                  dec.v_cache, c4.slot_mapping), 8 * 256 + 256 * 4 * 1024 * 2,
        (lambda: tp.store_kvcache_torch(kt16, vt16, cache_t, cache_t, st4), 1.0,
         "torch index_copy_ scatter of the C4 tokens into a full-size host cache"),
        parity=store_rows_parity,
        rotated=lambda: store_copies(k.view(256, 8, 128), v.view(256, 8, 128), scratch_kc,
                                     scratch_vc, 1.0))
    del cache_t, scratch_kc, scratch_vc
    gu = c4.gate_up
    gun = _np(gu)
    gut = gu.cpu()
    act = torch.empty(256, 12288, dtype=torch.bfloat16, device=dev)
    add("C4", "silu_and_mul [256,2x12288]", lambda: ops.silu_and_mul(act, gu),
        256 * 3 * 12288 * 2,
        (lambda: tp.silu_and_mul_native(gut), 1.0,
         "torch SiluAndMul.forward_native on the full input"),
        parity=lambda: verdict(_np(act), oracle.silu_and_mul(gun, "bf16"), "bf16"),
        rotated=lambda: [lambda x_=x_, o_=o_: ops.silu_and_mul(o_, x_) for x_, o_ in
                         [(gu.clone(), torch.empty_like(act))
                          for _ in range(copies_for(256 * 3 * 12288 * 2))]])

    # The C4 chain end to end, in the engine's order (LlamaDecoderLayer.forward,
    # llama_decoder.py:34-42, without the GEMMs): add+RMSNorm -> rotary on q/k ->
    # store_kvcache -> paged decode of the rotated q -> SiLU-and-mul; once as the
    # separate ops, once with the store fused into the decode launch.
    hc, rc = c4.hidden.clone(), c4.residual.clone()
    qkv_c = c4.qkv.clone()
    qc, kc_, vc_ = qkv_c[:, :4096], qkv_c[:, 4096:5120], qkv_c[:, 5120:]
    dplan = ops.paged_decode_plan(256, 32, 8, 128, dec.max_seq_len, 0)
    dws = torch.zeros(max(1, dplan.workspace_bytes), dtype=torch.uint8, device=dev)
    dout = torch.empty(256, 32, 128, dtype=torch.bfloat16, device=dev)
    act_c = torch.empty(256, 12288, dtype=torch.bfloat16, device=dev)

    def chain(fused):
        ops.fused_add_rms_norm(hc, rc, c4.norm_weight, 1e-6)
        ops.rotary_embedding(c4.positions, qc, kc_, 128, rope.cos_sin_cache, True)
        if fused:
            ops.store_paged_decode(dout, qc.view(256, 32, 128), kc_.view(256, 8, 128),
                                   vc_.view(256, 8, 128), dec.k_cache, dec.v_cache,
                                   c4.slot_mapping, dec.block_tables, dec.ctx_lens, dec.scale,
                                   dplan.part_tokens, dplan.max_parts, dws)
        else:
            ops.store_kvcache(kc_.view(256, 8, 128), vc_.view(256, 8, 128), dec.k_cache,
                              dec.v_cache, c4.slot_mapping)
            ops.paged_decode(dout, qc.view(256, 32, 128), dec.k_cache, dec.v_cache,
                             dec.block_tables, dec.ctx_lens, dec.scale, dplan.part_tokens,
                             dplan.max_parts, dws)
        ops.silu_and_mul(act_c, gu)

    chain_bytes = ((4 * 256 * 4096 + 4096) * 2 + 2 * 256 * 5120 * 2 + 256 * 8 + 256 * 128 * 4
                   + 8 * 256 + 256 * 4 * 1024 * 2 + dec.algorithmic_bytes()
                   + 256 * 3 * 12288 * 2)
    add("C4", "chain: add+RMSNorm, rotary, store_kvcache, paged_decode, silu_and_mul "
              "(separate launches)", lambda: chain(False), chain_bytes, iters=30)
    add("C4", "chain with the store fused into the decode (store_paged_decode)",
        lambda: chain(True), chain_bytes, iters=30)

    def decode_cpu(case, nseq):
        """The reference's torch decode path (oracle.torch_path.decode_torch: page gather,
        repeat_interleave, SDPA in bf16; fp8 pages dequantised per kv head) on nseq
        sequences (shortest..longest spread; all of them when nseq >= batch), their pages
        copied to the host first; and the numpy oracle on the same sequences for the
        parity verdict."""
        from oracle.torch_path import decode_torch

        ctx = case.ctx_lens.cpu().numpy().astype(np.int64)
        bt = case.block_tables.cpu().numpy()
        bs = case.k_cache.shape[1]
        order = np.argsort(ctx)
        pick = (list(range(len(ctx))) if nseq >= len(ctx) else
                sorted(set(order[np.linspace(0, len(ctx) - 1, nseq).astype(int)].tolist())))
        qh = case.q.cpu()
        fp8 = case.k_cache.dtype == torch.float8_e4m3fn
        ks = None if case.k_scale is None else case.k_scale.cpu()
        vs = None if case.v_scale is None else case.v_scale.cpu()
        data = []
        for i in pick:
            n = int(ctx[i])
            ids = torch.from_numpy(bt[i, :(n + bs - 1) // bs].astype(np.int64)).to(dev)
            data.append((i, n, case.k_cache[ids].cpu(), case.v_cache[ids].cpu()))
        data.sort(key=lambda e: e[1])  # by length, so `check` below spans short to long

        def run_torch():
            for i, n, kp, vp in data:
                decode_torch(qh[i:i + 1], kp, vp, torch.tensor([n]),
                             torch.arange(kp.shape[0])[None], case.scale, k_scale=ks, v_scale=vs)

        # The parity verdict: the numpy oracle on up to 4 of those sequences (shortest,
        # longest and two between).
        check = [data[j] for j in sorted(set(np.linspace(0, len(data) - 1,
                                                         min(4, len(data))).astype(int)))]

        def run_oracle():
            ksn = None if ks is None else ks.numpy()
            vsn = None if vs is None else vs.numpy()
            qn = _np(case.q)
            return [i for i, _, _, _ in check], np.concatenate([
                oracle.paged_decode(qn[i:i + 1],
                                    kp.view(torch.uint8).numpy() if fp8 else kp.float().numpy(),
                                    vp.view(torch.uint8).numpy() if fp8 else vp.float().numpy(),
                                    np.arange(kp.shape[0])[None], np.array([n]), case.scale,
                                    ksn, vsn) for i, n, kp, vp in check])

        frac = sum(n for _, n, _, _ in data) / float(ctx.sum())
        where = ("the whole batch" if len(pick) == len(ctx) else
                 f"{len(pick)} of {len(ctx)} sequences ({frac * 100:.1f}% of the cached tokens), "
                 "scaled to the batch")
        return (run_torch, frac, "oracle.torch_path.decode_torch (the reference's _decode_torch, "
                                 f"attention_impl.py:592-664) on {where}"), run_oracle

    decode_refs = {}

    def decode_parity(name, out, oracle_fn):
        """The oracle's rows for the sampled sequences (computed once per configuration)
        against the same rows of the GPU output, rounded to bf16 as the baseline's."""
        if name not in decode_refs:
            decode_refs[name] = oracle_fn()
        pick, ref = decode_refs[name]
        return verdict(_np(out)[pick], oracle.round_to(ref, "bf16"), "bf16")

    for t, hh in ((64, 32), (8192, 32)):
        g = torch.Generator().manual_seed(workloads.SEED)
        po = torch.randn(t, hh, 128, generator=g).to(torch.bfloat16).to(dev)
        so = torch.randn(t, hh, 128, generator=g).to(torch.bfloat16).to(dev)
        pl = (3 * torch.randn(hh, t, generator=g)).to(dev)
        sl = (3 * torch.randn(hh, t, generator=g)).to(dev)
        mo, ml = torch.empty_like(po), torch.empty_like(pl)
        arrs = [_np(x) for x in (po, pl, so, sl)]
        add("merge", f"merge_attn_states bf16 [{t},{hh},128] + lse",
            lambda po=po, pl=pl, so=so, sl=sl, mo=mo, ml=ml:
            ops.merge_attn_states(mo, po, pl, so, sl, ml),
            3 * t * hh * 128 * 2 + 3 * hh * t * 4,
            (lambda arrs=arrs: oracle.merge_attn_states(*arrs, "bf16"), 1.0,
             "oracle.merge_attn_states on the full input"),
            parity=lambda mo=mo, ml=ml, arrs=arrs: verdict(
                (_np(mo), _np(ml)), oracle.merge_attn_states(*arrs, "bf16"), ["bf16", "f32"]),
            rotated=(lambda po=po, pl=pl, so=so, sl=sl, t=t, hh=hh: [
                lambda a=a: ops.merge_attn_states(*a) for a in [
                    (torch.empty_like(po), po.clone(), pl.clone(), so.clone(), sl.clone(),
                     torch.empty_like(pl))
                    for _ in range(copies_for(3 * t * hh * 128 * 2 + 3 * hh * t * 4))]])
            if t <= 1024 else None)

    c3 = workloads.c3_decode(dev)
    c5 = workloads.c5_fp8_decode(dev)
    cpu_legs, oracle_legs = {}, {}
    # C3's batch and context lengths at the other head shapes the reference builds the
    # decode op with: Qwen3-Next's full attention (qwen3_next_attention.py:148-150),
    # Whisper large's (whisper_attention.py:185-190) and a gpt-oss-like group of 8.
    shapes = (("Qwen3-Next heads", 16, 2, 256), ("Whisper heads", 20, 20, 64),
              ("gpt-oss-like heads", 64, 8, 64))
    # C3 at the page sizes the reference engine picks besides 256: 16 tokens
    # (AttnBackendConfig.auto_detect for capability major 9, infra/context.py:68-73,
    # which PyTorch-ROCm reports for gfx950) and 64, over a pool of the same bytes.
    pages = (("C3 16-token pages", 16), ("C3 64-token pages", 64))
    for name, case, splits, nseq in (("C4", dec, 0, 256), ("C3", c3, 0, 64), ("C5", c5, 0, 1),
                                     ("C5", c5, 16, 0), ("C5", c5, 32, 0), ("C5", c5, 64, 0),
                                     *((n, (32, 8, 128, bs_), 0, 4) for n, bs_ in pages),
                                     *((n, (hq_, hk_, d_, 256), 0, 4) for n, hq_, hk_, d_ in shapes)):
        if isinstance(case, tuple):  # C3's lengths at another head shape or page size
            del out, ws
            torch.cuda.empty_cache()
            case = workloads.c3_decode(dev, num_heads=case[0], kv_heads=case[1],
                                       head_dim=case[2], block_size=case[3],
                                       pool_blocks=4096 * 256 // case[3])
        b, hq, d = case.q.shape
        hk = case.k_cache.shape[2]
        part, nparts, wsb = ops.paged_decode_plan(b, hq, hk, d, case.max_seq_len, splits)
        ws = torch.zeros(max(1, wsb), dtype=torch.uint8, device=dev)
        out = torch.empty_like(case.q)
        if nseq:
            cpu_legs[name], oracle_legs[name] = decode_cpu(case, nseq)
        add(name, f"paged_decode {str(case.k_cache.dtype).replace('torch.', '')} B={b} Hq={hq} "
                  + (f"Hk={hk} D={d} " if d != 128 else "")
                  + (f"block={case.k_cache.shape[1]} " if case.k_cache.shape[1] != 256 else "")
                  + f"{'balanced' if part == 0 else f'{nparts} partitions'}",
            lambda: ops.paged_decode(out, case.q, case.k_cache, case.v_cache, case.block_tables,
                                     case.ctx_lens, case.scale, part, nparts, ws, case.k_scale,
                                     case.v_scale), case.algorithmic_bytes(),
            cpu_legs[name] if nseq else None, iters=30,
            parity=lambda name=name, out=out: decode_parity(name, out, oracle_legs[name]))
    del case, out, ws
    torch.cuda.empty_cache()
    # C3 at 256-, 16- and 64-token pages timed in alternation: six rounds of 10 calls
    # of each (every call after the flush), so that the page sizes see the same
    # clocks; the rows above time each once, minutes apart.
    ilv_cases = {bs_: workloads.c3_decode(dev, block_size=bs_, pool_blocks=4096 * 256 // bs_)
                 for bs_ in (256, 16, 64)}
    ilv_fns, ilv_keep, ilv_us = {}, [], {bs_: [] for bs_ in ilv_cases}
    for bs_, cs in ilv_cases.items():
        b_, hq_, d_ = cs.q.shape
        part_, np_, wsb_ = ops.paged_decode_plan(b_, hq_, cs.k_cache.shape[2], d_, cs.max_seq_len, 0)
        ws_ = torch.zeros(max(1, wsb_), dtype=torch.uint8, device=dev)
        out_ = torch.empty_like(cs.q)
        ilv_keep.append((ws_, out_))
        ilv_fns[bs_] = (lambda cs=cs, out_=out_, ws_=ws_, part_=part_, np_=np_: ops.paged_decode(
            out_, cs.q, cs.k_cache, cs.v_cache, cs.block_tables, cs.ctx_lens, cs.scale, part_,
            np_, ws_))
    for _ in range(6):
        for bs_, fn_ in ilv_fns.items():
            ilv_us[bs_].append(time_call(fn_, iters=10, warmup=2, flush=flush)[0] * 1e3)
    ilv_row = {"config": "C3 page sizes", "op": "paged_decode bfloat16 B=64 Hq=32 at 256-, 16- "
               "and 64-token pages, timed in alternation (6 rounds x 10 calls each)",
               "us_median": {}, "frac_of_8TBs": {}, "ratio_to_256": {}}
    for bs_, us_ in ilv_us.items():
        med_ = statistics.median(us_)
        nb_ = ilv_cases[bs_].algorithmic_bytes()
        ilv_row["us_median"][str(bs_)] = round(med_, 2)
        ilv_row["frac_of_8TBs"][str(bs_)] = round(nb_ / (med_ * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
        ilv_row["ratio_to_256"][str(bs_)] = round(med_ / statistics.median(ilv_us[256]), 4)
    rows.append(ilv_row)
    print(json.dumps(ilv_row), file=sys.stderr, flush=True)
    del ilv_cases, ilv_fns, ilv_keep
    torch.cuda.empty_cache()
    # Prefill (FlashAttnPrefill with a block table) at Qwen3-8B heads, with torch's
    # own SDPA (flash backend, dense contiguous K/V) on the same GPU beside it.
    pf_cases = [(label, ql, kl, 32, 8, 128, False) for label, ql, kl in PREFILL_CASES]
    pf_cases += [("1x2048 prompt", [2048], [2048], hq_, hk_, d_, False)
                 for _, hq_, hk_, d_ in shapes[:2]]
    # fp8 e4m3fn pages (per-kv-head scales), dequantised exactly in the kernel.
    pf_cases += [(label, ql, kl, 32, 8, 128, True) for label, ql, kl in PREFILL_CASES[:2]]
    pf_cases = [c_ + (True,) for c_ in pf_cases]
    # One chunk over a long cache (128 work-groups): the work-group key split spreads
    # each block's keys over several work-groups; the launch without it beside it.
    pf_cases += [("1x512 chunk over 8192", [512], [8192], 32, 8, 128, False, sp_)
                 for sp_ in (True, False)]
    for label, ql, kl, hq_, hk_, d_, fp8, split_ in pf_cases:
        q, kc, vc, bt, cu_q, cu_k, mq, flop = prefill_case(dev, ql, kl, workloads.SEED + 11,
                                                           hq_, hk_, d_)
        ks = vs = None
        if fp8:
            gs = torch.Generator().manual_seed(workloads.SEED + 13)
            ks = (0.01 + 0.09 * torch.rand(hk_, generator=gs)).float().to(dev)
            vs = (0.01 + 0.09 * torch.rand(hk_, generator=gs)).float().to(dev)
            kc = workloads.quantize_fp8(kc.float(), ks)
            vc = workloads.quantize_fp8(vc.float(), vs)
        pout = torch.empty_like(q)
        ops.PREFILL_SPLIT = split_
        try:
            med, _ = time_call(lambda: ops.paged_prefill(pout, q, kc, vc, bt, cu_q, cu_k, mq,
                                                         d_ ** -0.5, ks, vs,
                                                         max_seqlen_k=max(kl)),
                               iters=20, warmup=3, flush=flush)
        finally:
            ops.PREFILL_SPLIT = True
        heads = f"Hq={hq_} Hk={hk_}" + (f" D={d_}" if d_ != 128 else "")
        row = {"config": "prefill",
               "op": f"paged_prefill {'fp8' if fp8 else 'bf16'} {heads} {label}" +
                     ("" if split_ else " (without the work-group key split)"),
               "us_median": round(med * 1e3, 2), "flop": flop,
               "TFLOPs": round(flop / (med * 1e-3) / 1e12, 1),
               "frac_of_2.5PFLOPs": round(flop / (med * 1e-3) / 2.5e15, 4)}
        rows.append(row)
        print(json.dumps(row), file=sys.stderr, flush=True)
    try:  # torch's flash SDPA on dense [1, 32, 2048, 128] bf16 (MHA-expanded K/V)
        from torch.nn.attention import SDPBackend, sdpa_kernel
        g = torch.Generator().manual_seed(workloads.SEED + 12)
        tq, tk, tv = (torch.randn(1, 32, 2048, 128, generator=g).to(torch.bfloat16).to(dev)
                      for _ in range(3))
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
            med, _ = time_call(lambda: torch.nn.functional.scaled_dot_product_attention(
                tq, tk, tv, is_causal=True), iters=20, warmup=3, flush=flush)
        flop = 2048 * 2049 // 2 * 32 * 4 * 128
        row = {"config": "prefill", "op": "torch SDPA flash backend, dense 1x2048 causal (comparison)",
               "us_median": round(med * 1e3, 2), "flop": flop,
               "TFLOPs": round(flop / (med * 1e-3) / 1e12, 1),
               "frac_of_2.5PFLOPs": round(flop / (med * 1e-3) / 2.5e15, 4)}
        rows.append(row)
        print(json.dumps(row), file=sys.stderr, flush=True)
    except Exception as e:  # noqa: BLE001 - the comparison row is optional
        print(f"torch SDPA flash comparison skipped: {e!r}", file=sys.stderr, flush=True)

    # Decode step of Attention.forward_impl at C3: store + decode as two calls, and fused.
    rows3 = workloads.decode_step_rows(c3)
    b3, hq3, d3 = c3.q.shape
    part3, np3, wsb3 = ops.paged_decode_plan(b3, hq3, c3.k_cache.shape[2], d3, c3.max_seq_len, 0)
    ws3 = torch.zeros(max(1, wsb3), dtype=torch.uint8, device=dev)
    out3 = torch.empty_like(c3.q)
    step_bytes = c3.algorithmic_bytes() + b3 * (4 * rows3.key[0].numel() * 2 + 8)

    def two_calls():
        ops.store_kvcache(rows3.key, rows3.value, c3.k_cache, c3.v_cache, rows3.slot_mapping)
        ops.paged_decode(out3, c3.q, c3.k_cache, c3.v_cache, c3.block_tables, c3.ctx_lens,
                         c3.scale, part3, np3, ws3)

    def fused():
        ops.store_paged_decode(out3, c3.q, rows3.key, rows3.value, c3.k_cache, c3.v_cache,
                               rows3.slot_mapping, c3.block_tables, c3.ctx_lens, c3.scale, part3,
                               np3, ws3)

    add("C3", "decode step: store_kvcache + paged_decode (two calls)", two_calls, step_bytes,
        iters=30)
    add("C3", "decode step: store_paged_decode (fused)", fused, step_bytes, iters=30)
    if limiter is not None:
        limiter.__exit__(None, None, None)
    if args.table_json:
        Path(args.table_json).parent.mkdir(parents=True, exist_ok=True)
        Path(args.table_json).write_text(json.dumps(rows, indent=1))
    return rows


# The prefill rows of the per-op table: (label, query lengths, key lengths).
PREFILL_CASES = (("1x2048 prompt", [2048], [2048]),
                 ("4x512 chunks over 4096", [512] * 4, [4096] * 4),
                 ("16x512 prompts", [512] * 16, [512] * 16))


def prefill_case(dev, q_lens, k_lens, seed, hq=32, hk=8, d=128):
    """Paged prefill inputs (default Qwen3-8B heads: Hq 32, Hk 8, head 128; 256-token
    pages from a seeded permutation), and the FLOPs of the visible (query, key) pairs."""
    import numpy as np
    import torch

    g = torch.Generator().manual_seed(seed)
    bs = 256
    pages = [(k + bs - 1) // bs for k in k_lens]
    nb = sum(pages)
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    bt = torch.full((len(k_lens), max(pages)), -1, dtype=torch.int32)
    off = 0
    for i, p in enumerate(pages):
        bt[i, :p] = perm[off:off + p]
        off += p
    cu_q = torch.tensor([0] + list(np.cumsum(q_lens)), dtype=torch.int32, device=dev)
    cu_k = torch.tensor([0] + list(np.cumsum(k_lens)), dtype=torch.int32, device=dev)
    q = torch.randn(sum(q_lens), hq, d, generator=g).to(torch.bfloat16).to(dev)
    kc = torch.randn(nb, bs, hk, d, generator=g).to(torch.bfloat16).to(dev)
    vc = torch.randn(nb, bs, hk, d, generator=g).to(torch.bfloat16).to(dev)
    visible = sum(sum(max(0, min(kl, kl - ql + j + 1)) for j in range(ql))
                  for ql, kl in zip(q_lens, k_lens))
    return q, kc, vc, bt.to(dev), cu_q, cu_k, max(q_lens), visible * hq * 4 * d


def profile_prefill(reps: int = 3):
    """The per-op table's prefill cases, `reps` calls each, every call after a 512 MB
    read that evicts L2 and the MALL: the program rocprofv3 --pmc / --kernel-trace runs
    for the prefill kernel's counters.  Prints one JSON line per case."""
    import torch

    from fastkernels_amd import ops, workloads

    dev = torch.device("cuda:0")
    flush = _flush_buffer(dev)
    for label, ql, kl in PREFILL_CASES:
        q, kc, vc, bt, cu_q, cu_k, mq, flop = prefill_case(dev, ql, kl, workloads.SEED + 11)
        out = torch.empty_like(q)
        for _ in range(reps):
            flush.sum()
            ops.paged_prefill(out, q, kc, vc, bt, cu_q, cu_k, mq, 128 ** -0.5,
                              max_seqlen_k=max(kl))
        torch.cuda.synchronize()
        print(json.dumps({"case": label, "flop": flop, "calls": reps}), flush=True)


def profile_ops(reps: int = 3):
    """Each op of the decode step on its C1-C5 inputs, `reps` times, every call after a
    512 MB read that evicts L2 and the MALL: the program rocprofv3 --pmc runs to count
    the HBM bytes (FETCH_SIZE / WRITE_SIZE) each kernel moves per dispatch.  Prints one
    JSON line per op: its kernels' name fragment and algorithmic bytes per call."""
    import torch

    from fastkernels_amd import ops, workloads
    from fastkernels_amd.candidate.L1.rotary_emb import RotaryEmbedding

    dev = torch.device("cuda:0")
    flush = _flush_buffer(dev)
    rows = []

    def run(op, kernel, nbytes, fn):
        for _ in range(reps):
            flush.sum()
            fn()
        torch.cuda.synchronize()
        rows.append({"op": op, "kernel": kernel, "algorithmic_bytes": nbytes, "calls": reps})
        print(json.dumps(rows[-1]), flush=True)

    c1 = workloads.c1_norm(dev)
    run("C1 fused_add_rmsnorm bf16 [256,1024]", "fused_add_rmsnorm", (4 * 256 * 1024 + 1024) * 2,
        lambda: ops.fused_add_rms_norm(c1.x, c1.residual, c1.weight, c1.eps))
    c2 = workloads.c2_store(dev)
    nvalid = int((c2.slot_mapping >= 0).sum().item())
    run("C2 store_kvcache [4096,8,128]", "store_kvcache", 8 * 4096 + nvalid * 4 * 8 * 128 * 2,
        lambda: ops.store_kvcache(c2.key, c2.value, c2.k_cache, c2.v_cache, c2.slot_mapping))
    del c2
    c4 = workloads.c4_chain(dev)
    run("C4 fused_add_rmsnorm bf16 [256,4096]", "fused_add_rmsnorm", (4 * 256 * 4096 + 4096) * 2,
        lambda: ops.fused_add_rms_norm(c4.hidden, c4.residual, c4.norm_weight, 1e-6))
    rope = RotaryEmbedding(128, c4.max_position, c4.rope_theta).to(dev)
    q, k, v = c4.qkv[:, :4096], c4.qkv[:, 4096:5120], c4.qkv[:, 5120:]
    run("C4 rotary q[256,32x128] k[256,8x128]", "rotary",
        2 * 256 * 5120 * 2 + 256 * 8 + 256 * 128 * 4,
        lambda: ops.rotary_embedding(c4.positions, q, k, 128, rope.cos_sin_cache, True))
    dec = c4.decode
    run("C4 store_kvcache [256,8,128]", "store_kvcache", 8 * 256 + 256 * 4 * 1024 * 2,
        lambda: ops.store_kvcache(k.view(256, 8, 128), v.view(256, 8, 128), dec.k_cache,
                                  dec.v_cache, c4.slot_mapping))
    act = torch.empty(256, 12288, dtype=torch.bfloat16, device=dev)
    run("C4 silu_and_mul [256,2x12288]", "silu_and_mul", 256 * 3 * 12288 * 2,
        lambda: ops.silu_and_mul(act, c4.gate_up))
    g = torch.Generator().manual_seed(workloads.SEED + 7)
    qw = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16).to(dev)
    kw = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16).to(dev)
    qk_bytes = (256 * (4096 + 2 * 1024) * 2 + 256 * (4096 + 1024) * 2 + 256 * 2 * 1024 * 2
                + 256 * 16 + 256 * 128 * 4 + 2 * 128 * 2)
    run("C4 qk_norm_rope_store", "qk_norm_rope_store", qk_bytes,
        lambda: ops.qk_norm_rope_store(c4.positions, q, k, v, dec.k_cache, dec.v_cache,
                                       c4.slot_mapping, 128, rope.cos_sin_cache, True, qw, kw,
                                       1e-6))
    for name, case in (("C4", dec), ("C5", None)):
        if case is None:
            del c4, dec
            torch.cuda.empty_cache()
            case = workloads.c5_fp8_decode(dev)
        b, hq, d = case.q.shape
        plan = ops.paged_decode_plan(b, hq, case.k_cache.shape[2], d, case.max_seq_len, 0)
        ws = torch.zeros(max(1, plan.workspace_bytes), dtype=torch.uint8, device=dev)
        out = torch.empty_like(case.q)
        total = case.algorithmic_bytes()
        run(f"{name} paged_decode {str(case.k_cache.dtype).replace('torch.', '')} B={b} Hq={hq} "
            "balanced (main kernel; the merge is listed separately)", "paged_decode_balanced",
            total - out.numel() * out.element_size(),
            lambda case=case, plan=plan, ws=ws, out=out: ops.paged_decode(
                out, case.q, case.k_cache, case.v_cache, case.block_tables, case.ctx_lens,
                case.scale, plan.part_tokens, plan.max_parts, ws, case.k_scale, case.v_scale))
    return rows


def calib_copy():
    import torch

    dev = torch.device("cuda:0")
    src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calib_copy_bytes": src.numel(), "launches": 5}), flush=True)


def main():
    args = _parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the decode path has no cross-GPU "
              "exchange in this tier); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    from fastkernels_amd import _native

    _native.lib()
    if args.calib_copy:
        calib_copy()
        return
    if args.profile_ops:
        profile_ops()
        return
    if args.profile_prefill:
        profile_prefill()
        return
    if args.table:
        bench_table(args)
        return
    result, case, out = bench_decode(args)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline_decode(case, args.cpu_seconds, gpu_out=out)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
