"""Candidates ``StoreKVCache`` and ``StoreKVCacheHND`` for
fastkernels/tasks/baseline/L1/store_kvcache.py:71-99.

``forward(key, value, k_cache, v_cache, slot_mapping)`` scatters each token's
[num_kv_heads, head_dim] K and V rows into the NHD paged caches
[num_blocks, block_size, num_kv_heads, head_dim] at ``slot_mapping[i]``,
skipping slots < 0, and returns None, exactly as the Triton
``_store_kvcache_kernel`` (store_kvcache.py:16-35).  int32 and int64 slot
mappings are read natively (no conversion tensor is allocated), and slots past
the end of the cache are skipped instead of written.  A key/value dtype that
differs from the cache's (e.g. bf16 rows into a float8_e4m3fn cache) is converted
as the Triton store's implicit cast does: round to nearest even, fp8 saturating
at +-448.

``StoreKVCacheHND(page_size)`` writes the same rows into HND caches
[num_blocks, num_kv_heads, page_size, head_dim], head h of token i at
``[slot // page_size, h, slot % page_size]``, as ``_store_kvcache_hnd_kernel``
(store_kvcache.py:36-68); key and cache dtypes must match there.
"""
from __future__ import annotations

import sys
from pathlib import Path

import torch
import torch.nn as nn

try:
    import fastkernels_amd  # noqa: F401
except ImportError:  # loaded by file path from the reference harness
    sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
from fastkernels_amd import ops


class StoreKVCache(nn.Module):
    """NHD layout store: [num_blocks, block_size, num_kv_heads, head_dim]."""

    def forward(self, key, value, k_cache, v_cache, slot_mapping):
        if torch.compiler.is_compiling():
            torch.ops.fastkernels_amd.store_kvcache(key, value, k_cache, v_cache, slot_mapping)
        else:
            ops.store_kvcache(key, value, k_cache, v_cache, slot_mapping)


class StoreKVCacheHND(nn.Module):
    """HND layout store: [num_blocks, num_kv_heads, block_size, head_dim]."""

    def __init__(self, page_size: int):
        super().__init__()
        self.page_size = page_size

    def forward(self, key, value, k_cache, v_cache, slot_mapping):
        if torch.compiler.is_compiling():
            torch.ops.fastkernels_amd.store_kvcache_hnd(key, value, k_cache, v_cache,
                                                        slot_mapping, self.page_size)
        else:
            ops.store_kvcache_hnd(key, value, k_cache, v_cache, slot_mapping, self.page_size)
