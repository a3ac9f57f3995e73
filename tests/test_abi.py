"""The C ABI without a GPU: libfk_amd.so loads, exports every symbol the header
declares, and its host-side logic (planning, argument validation) behaves.

Only calls that return before any HIP launch are made here (argument errors and
the host-only planner), so these tests run on a machine without a GPU.
"""
from __future__ import annotations

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "fastkernels_amd.h"


@pytest.fixture(scope="module")
def lib():
    from fastkernels_amd import _native, build

    if not _native.LIB_PATH.exists():
        build.build(verbose=False)
    return _native.lib()


def header_symbols() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fk_\w+)\s*\(", text)))


def test_header_declares_the_operator_set():
    syms = header_symbols()
    for name in ("fk_rmsnorm", "fk_fused_add_rmsnorm", "fk_rotary_embedding", "fk_store_kvcache",
                 "fk_paged_decode_plan", "fk_paged_decode", "fk_paged_decode_partials",
                 "fk_paged_decode_reduce", "fk_silu_and_mul", "fk_version", "fk_last_error"):
        assert name in syms


def test_library_exports_every_header_symbol(lib):
    from fastkernels_amd import _native

    for name in header_symbols():
        assert hasattr(lib, name), f"{name} declared but not exported"
        assert name in _native.EXPORTED, f"{name} has no ctypes signature"
    if shutil.which("nm"):
        out = subprocess.run(["nm", "-D", "--defined-only", str(_native.LIB_PATH)],
                             capture_output=True, text=True, check=True).stdout
        exported = set(re.findall(r"\sT\s+(fk_\w+)$", out, flags=re.M))
        assert set(header_symbols()) <= exported
        # nothing outside the header leaks as an fk_ entry point
        assert exported <= set(header_symbols())


def test_version_and_clean_error(lib):
    from fastkernels_amd import _native

    # Major version 2: fk_paged_prefill / fk_varlen_prefill took head_size_v, lse and
    # lse_row_stride; the bindings refuse a library of another major version.
    assert lib.fk_version() // 10000 == _native.ABI_MAJOR == 2
    text = HEADER.read_text()
    assert re.search(r"#define FK_VERSION_MAJOR 2\b", text)


def test_prefill_head_sizes_and_lse_arguments(lib):
    """fk_varlen_prefill refuses head-size pairs that are not built (before any launch)
    and names them; the Python layer's table agrees with the C library's."""
    from fastkernels_amd import _native as N
    from fastkernels_amd import ops

    fake = ctypes.c_void_p(0x100000)
    cu = ctypes.c_void_p(0x200000)

    def varlen(d, dv, lse_stride=0):
        return lib.fk_varlen_prefill(fake, 8 * dv, fake, 8 * d, fake, 2 * d, fake, 2 * dv,
                                     cu, cu, 1, 16, 16, 8, 2, d, dv, 0.1, 1, -1, None,
                                     fake if lse_stride else None, lse_stride, None)

    for d, dv in ((48, 48), (128, 64), (192, 192), (512, 512), (80, 72)):
        assert not ops.prefill_heads_supported(d, dv)
        assert varlen(d, dv) == N.FK_ERR_UNSUPPORTED, (d, dv)
        assert "head sizes" in _last_error(lib)
    for d, dv in ((80, 80), (192, 128), (72, 72), (32, 32), (96, 96)):
        assert ops.prefill_heads_supported(d, dv)
    assert not ops.prefill_heads_supported(80, 80, fp8=True)
    assert ops.prefill_heads_supported(128, 128, fp8=True)
    assert varlen(128, 128, lse_stride=-1) == N.FK_ERR_INVALID_ARG


def test_prefill_page_bytes_bound(lib):
    """fk_paged_prefill addresses a page's rows by 32-bit offsets from its first row, so
    it refuses pages of 2^32 bytes or more (before any launch); one byte less per page
    passes that check."""
    from fastkernels_amd import _native as N

    fake = ctypes.c_void_p(0x100000)
    cu = ctypes.c_void_p(0x200000)

    def paged(block_size, hk, d):
        return lib.fk_paged_prefill(fake, 32 * d, fake, 32 * d, fake, fake, N.FK_DTYPE_BF16,
                                    None, None, fake, 4, cu, cu, 1, 0, 0, 32, hk, d, d,
                                    block_size, 1, 0.1, 1, -1, None, None)

    # 2^22 slots of 8 heads x 128 bf16 (2 KiB rows): 2^33 bytes per page
    assert paged(1 << 22, 8, 128) == N.FK_ERR_INVALID_ARG
    assert "2^32" in _last_error(lib)
    # 2^20 slots of 2 KiB rows: 2^31 bytes; max_seqlen_q 0 then returns before launching
    assert paged(1 << 20, 8, 128) == N.FK_OK


def _last_error(lib) -> str:
    return lib.fk_last_error().decode()


def test_plan_host_logic(lib):
    from fastkernels_amd import _native

    part, nparts, ws = _native.plan(64, 32, 8, 128, 8192, 0)
    assert part == 0 and nparts >= 1  # balanced: one range per work-group
    rows = nparts * 2 * 32
    assert ws >= rows * 128 * 4 + rows * 8 + (64 + 2) * 4
    part, nparts, ws = _native.plan(64, 32, 8, 128, 8192, 16)
    assert (part, nparts) == (512, 16)
    part, nparts, _ = _native.plan(8, 64, 8, 128, 131072, 64)
    assert (part, nparts) == (2048, 64)
    part, nparts, _ = _native.plan(4, 32, 8, 128, 100, 3)  # rounds up to 64-token units
    assert part == 64 and nparts == 2
    part, nparts, _ = _native.plan(10000, 32, 8, 128, 4096, 0)  # too many for LDS prefix sums
    assert part > 0
    # head sizes 64 / 256: partial rows of head_size floats
    _, n64, ws64 = _native.plan(64, 32, 8, 64, 8192, 0)
    _, n256, ws256 = _native.plan(64, 32, 8, 256, 8192, 0)
    assert n64 == n256 and ws256 - ws64 >= n64 * 2 * 32 * (256 - 64) * 4
    # Balanced group counts, relative to C3's (8 kv heads: one work-group per CU).
    # Fewer than 8 virtual heads: 4 / Hk work-groups per CU, whatever the group size
    # (a group above 16 query heads takes one wave per 16 query columns).
    _, n_c3, _ = _native.plan(64, 32, 8, 128, 8192, 0)
    _, n_g32, _ = _native.plan(64, 64, 2, 128, 8192, 0)  # 2 kv heads x 2 column blocks
    _, n_g8, _ = _native.plan(64, 16, 2, 128, 8192, 0)   # 2 kv heads x 1 column block
    assert n_g8 == n_g32 == 2 * n_c3
    assert _native.plan(64, 8, 1, 128, 8192, 0)[1] == 4 * n_c3
    assert _native.plan(64, 16, 4, 128, 8192, 0)[1] == n_c3
    # Several full groups of 8 virtual heads: one work-group per CU over all of them;
    # a last group with idle waves keeps one per CU per group.
    assert _native.plan(16, 32, 32, 128, 8192, 0)[1] * 4 == n_c3
    assert _native.plan(64, 20, 20, 64, 8192, 0)[1] == n_c3
    with pytest.raises(_native.FkError, match="head_size"):
        _native.plan(64, 32, 8, 96, 8192, 0)
    with pytest.raises(_native.FkError):
        _native.plan(-1, 32, 8, 128, 10, 0)


def test_argument_errors_return_before_launch(lib):
    from fastkernels_amd import _native as N

    fake = ctypes.c_void_p(0x100000)  # never dereferenced: every call below is rejected first
    stream = ctypes.c_void_p(0)
    rc = lib.fk_store_kvcache(fake, 8, fake, 8, fake, fake, fake, 1, 4, 8, 3, 64, stream)
    assert rc == N.FK_ERR_INVALID_ARG and "elem_bytes" in _last_error(lib)
    rc = lib.fk_store_kvcache(fake, 4, fake, 8, fake, fake, fake, 1, 4, 8, 2, 64, stream)
    assert rc == N.FK_ERR_INVALID_ARG and "stride" in _last_error(lib)
    rc = lib.fk_rmsnorm(fake, 64, fake, 64, fake, 2, 64, 1e-6, 9, stream)
    assert rc == N.FK_ERR_UNSUPPORTED and "dtype" in _last_error(lib)
    rc = lib.fk_fused_add_rmsnorm(fake, 32, fake, 64, fake, 2, 64, 1e-6, N.FK_DTYPE_BF16, stream)
    assert rc == N.FK_ERR_INVALID_ARG
    rc = lib.fk_rotary_embedding(fake, fake, 512, fake, 128, fake, 0, 100, 4, 4, 1, 128, 127, 1,
                                 N.FK_DTYPE_BF16, stream)
    assert rc == N.FK_ERR_INVALID_ARG and "rot_dim" in _last_error(lib)
    rc = lib.fk_silu_and_mul(fake, 4, fake, 4, -1, 2, N.FK_DTYPE_BF16, stream)
    assert rc == N.FK_ERR_INVALID_ARG

    def decode(**kw):
        a = dict(head=128, hq=32, hk=8, bs=256, nb=64, part=512, nparts=4, ws=fake, wsb=1 << 30,
                 kv=N.FK_DTYPE_BF16, window=-1)
        a.update(kw)
        return lib.fk_paged_decode(fake, a["hq"] * 128, fake, a["hq"] * 128, fake, fake, a["kv"],
                                   None, None, fake, 32, fake, 4, a["hq"], a["hk"], a["head"],
                                   a["bs"], a["nb"], 0.088, a["window"], None, a["part"],
                                   a["nparts"], a["ws"], a["wsb"], stream)

    assert decode(head=96) == N.FK_ERR_UNSUPPORTED and "head_size" in _last_error(lib)
    assert decode(head=512) == N.FK_ERR_UNSUPPORTED and "head_size" in _last_error(lib)
    assert decode(hq=30, hk=8) == N.FK_ERR_INVALID_ARG
    assert decode(bs=24) == N.FK_ERR_INVALID_ARG and "block_size" in _last_error(lib)
    assert decode(part=100) == N.FK_ERR_INVALID_ARG and "part_tokens" in _last_error(lib)
    assert decode(kv=N.FK_DTYPE_F32) == N.FK_ERR_INVALID_ARG
    assert decode(nb=0) == N.FK_ERR_INVALID_ARG and "block" in _last_error(lib)
    assert decode(wsb=16) == N.FK_ERR_WORKSPACE and "workspace" in _last_error(lib)
    assert decode(ws=None, part=0, nparts=256) == N.FK_ERR_WORKSPACE
    assert decode(window=-2) == N.FK_ERR_INVALID_ARG and "window_left" in _last_error(lib)


def test_python_layer_fails_loudly_without_gpu(lib):
    """No CPU fallback: CPU tensors are rejected, not computed."""
    import torch

    from fastkernels_amd import ops

    x = torch.zeros(4, 2 * 64, dtype=torch.bfloat16)
    out = torch.empty(4, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.silu_and_mul(out, x)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.rms_norm(torch.empty(4, 64), torch.zeros(4, 64), torch.ones(64), 1e-6)


def test_missing_library_raises(monkeypatch, tmp_path):
    from fastkernels_amd import _native

    monkeypatch.setattr(_native, "_lib", None)
    monkeypatch.setenv("FASTKERNELS_AMD_LIB", str(tmp_path / "absent.so"))
    with pytest.raises(RuntimeError, match="no fallback"):
        _native.lib()
    monkeypatch.setattr(_native, "_lib", None)
