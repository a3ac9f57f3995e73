"""ctypes binding of libfk_amd.so (the C ABI declared in include/fastkernels_amd.h).

The library is loaded from ``fastkernels_amd/_lib/libfk_amd.so`` (built in-tree
by ``python -m fastkernels_amd.build``).  There is no fallback: if the library
is missing or fails to load, :func:`lib` raises, so a GPU run can never silently
take another code path.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import c_float, c_int, c_int64, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libfk_amd.so"

FK_OK = 0
FK_ERR_INVALID_ARG = -1
FK_ERR_UNSUPPORTED = -2
FK_ERR_WORKSPACE = -3

# The C ABI's major version these bindings are written for (FK_VERSION_MAJOR in
# include/fastkernels_amd.h; fk_version() = 10000 * major + 100 * minor + patch).
ABI_MAJOR = 2

FK_DTYPE_F32 = 0
FK_DTYPE_F16 = 1
FK_DTYPE_BF16 = 2
FK_DTYPE_FP8_E4M3FN = 3

# name -> (restype, argtypes); mirrors include/fastkernels_amd.h.
_SIGNATURES = {
    "fk_version": (c_int, []),
    "fk_last_error": (ctypes.c_char_p, []),
    "fk_rmsnorm": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_int64,
                           c_float, c_int, c_void_p]),
    "fk_fused_add_rmsnorm": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                     c_int64, c_float, c_int, c_void_p]),
    "fk_rotary_embedding": (c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p,
                                    c_int, c_int64, c_int64, c_int, c_int, c_int, c_int, c_int,
                                    c_int, c_void_p]),
    "fk_store_kvcache": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p,
                                 c_void_p, c_int, c_int64, c_int64, c_int, c_int64, c_void_p]),
    "fk_store_kvcache_hnd": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p,
                                     c_void_p, c_int, c_int64, c_int, c_int, c_int, c_int,
                                     c_int64, c_void_p]),
    "fk_paged_decode_plan": (c_int, [c_int64, c_int, c_int, c_int, c_int64, c_int,
                                     ctypes.POINTER(c_int64), ctypes.POINTER(c_int64),
                                     ctypes.POINTER(c_int64)]),
    "fk_paged_decode": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int,
                                c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_int,
                                c_int, c_int, c_int, c_int64, c_float, c_int, c_void_p,
                                c_int64, c_int64, c_void_p, c_int64, c_void_p]),
    "fk_paged_decode_partials": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p,
                                         c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int64,
                                         c_void_p, c_int64, c_int, c_int, c_int, c_int, c_int64,
                                         c_float, c_int, c_void_p, c_int64, c_int64, c_void_p,
                                         c_int64, c_void_p]),
    "fk_paged_decode_reduce": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p,
                                       c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int64,
                                       c_void_p, c_int64, c_int, c_int, c_int, c_int, c_int64,
                                       c_float, c_int, c_void_p, c_int64, c_int64, c_void_p,
                                       c_int64, c_void_p]),
    "fk_paged_decode_noalloc": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p,
                                        c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int64,
                                        c_void_p, c_int64, c_int, c_int, c_int, c_int, c_int64,
                                        c_float, c_int, c_void_p, c_int64, c_int64, c_void_p]),
    "fk_silu_and_mul": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int64, c_int,
                                c_void_p]),
    "fk_store_paged_decode": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                      c_void_p, c_int64, c_void_p, c_int, c_void_p, c_void_p,
                                      c_int, c_void_p, c_void_p, c_void_p, c_int64, c_void_p,
                                      c_int64, c_int, c_int, c_int, c_int, c_int64, c_float,
                                      c_int, c_void_p, c_int64, c_int64, c_void_p, c_int64,
                                      c_void_p]),
    "fk_qk_norm_rope_store": (c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p,
                                      c_int64, c_void_p, c_void_p, c_float, c_void_p, c_int,
                                      c_int64, c_int, c_int, c_void_p, c_void_p, c_void_p, c_int,
                                      c_int64, c_int64, c_int, c_int, c_int, c_int, c_void_p]),
    "fk_paged_prefill": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int,
                                 c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p,
                                 c_int64, c_int64, c_int64, c_int, c_int, c_int, c_int, c_int,
                                 c_int64, c_float, c_int, c_int, c_void_p, c_void_p]),
    "fk_varlen_prefill": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                  c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_int64,
                                  c_int64, c_int, c_int, c_int, c_int, c_float, c_int, c_int,
                                  c_void_p, c_void_p, c_int64, c_void_p]),
    "fk_prefill_split_plan": (c_int, [c_int, c_int, c_int64, c_int64, c_int64, c_int64, c_int,
                                      c_int, c_int, c_int, c_int, ctypes.POINTER(c_int64)]),
    "fk_paged_prefill_ws": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p,
                                    c_int, c_void_p, c_void_p, c_void_p, c_int64, c_void_p,
                                    c_void_p, c_int64, c_int64, c_int64, c_int, c_int, c_int,
                                    c_int, c_int, c_int64, c_float, c_int, c_int, c_void_p,
                                    c_int64, c_void_p, c_int64, c_void_p]),
    "fk_varlen_prefill_ws": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                     c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_int64,
                                     c_int64, c_int, c_int, c_int, c_int, c_float, c_int, c_int,
                                     c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int64,
                                     c_void_p]),
    "fk_store_kvcache_convert": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_int, c_void_p,
                                         c_void_p, c_int, c_void_p, c_int, c_int64, c_int64,
                                         c_int64, c_void_p]),
    "fk_merge_attn_states": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p,
                                     c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int, c_int,
                                     c_int64, c_int, c_int, c_void_p, c_void_p]),
}

EXPORTED = tuple(_SIGNATURES)

_lib: ctypes.CDLL | None = None


class FkError(RuntimeError):
    """A libfk_amd entry point rejected its arguments or failed to launch."""

    def __init__(self, fn: str, code: int, message: str):
        super().__init__(f"{fn} failed with status {code}: {message}")
        self.code = code


def lib() -> ctypes.CDLL:
    """Load (once) and return the bound library; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    path = Path(os.environ.get("FASTKERNELS_AMD_LIB", str(LIB_PATH)))
    if not path.exists():
        raise RuntimeError(
            f"libfk_amd.so not found at {path}; build it with `python -m fastkernels_amd.build`"
            " (the HIP kernels are the only implementation; there is no fallback)")
    handle = ctypes.CDLL(str(path))
    handle.fk_version.restype = c_int
    handle.fk_version.argtypes = []
    version = handle.fk_version()
    if version // 10000 != ABI_MAJOR:
        raise RuntimeError(
            f"{path} implements C ABI version {version}, these bindings need major version "
            f"{ABI_MAJOR}: rebuild it with `python -m fastkernels_amd.build`")
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = handle
    return handle


def check(fn: str, code: int) -> None:
    if code != FK_OK:
        msg = lib().fk_last_error()
        raise FkError(fn, code, msg.decode() if msg else "")


def call(fn: str, *args) -> None:
    """Call entry point ``fn`` and raise FkError on a non-zero status."""
    check(fn, getattr(lib(), fn)(*args))


def prefill_split_bytes(paged: bool, kv_dtype: int, batch: int, total_q: int, max_seqlen_q: int,
                        max_seqlen_k: int, num_heads: int, num_kv_heads: int, head_size: int,
                        head_size_v: int, causal: bool) -> int:
    """fk_prefill_split_plan: the workspace bytes of the prefill's work-group key split
    (0: the launch does not split)."""
    ws = c_int64(0)
    check("fk_prefill_split_plan",
          lib().fk_prefill_split_plan(int(paged), kv_dtype, batch, total_q, max_seqlen_q,
                                      max_seqlen_k, num_heads, num_kv_heads, head_size,
                                      head_size_v, int(bool(causal)), ctypes.byref(ws)))
    return ws.value


def plan(batch: int, num_heads: int, num_kv_heads: int, head_size: int, max_seq_len: int,
         num_splits: int) -> tuple[int, int, int]:
    """fk_paged_decode_plan: (part_tokens, max_parts, workspace_bytes); part_tokens 0 is
    the length-balanced schedule."""
    part = c_int64(0)
    nparts = c_int64(0)
    ws = c_int64(0)
    check("fk_paged_decode_plan",
          lib().fk_paged_decode_plan(batch, num_heads, num_kv_heads, head_size, max_seq_len,
                                     num_splits, ctypes.byref(part), ctypes.byref(nparts),
                                     ctypes.byref(ws)))
    return part.value, nparts.value, ws.value
