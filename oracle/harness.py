"""The reference bench's paged-decode input fixer, restated for the tests.

TEST INFRASTRUCTURE ONLY (like the rest of ``oracle/``): the parity tests build
``FlashAttnDecode`` inputs the way the reference's ``fastkernels bench`` does
before timing a paged-decode candidate (``_fix_paged_decode``,
fastkernels/bench.py:1305-1329), and tests/test_harness_rules.py pins this
restatement with the assertions of the reference's own harness test
(tests/test_bench.py:285-316).  Nothing in ``fastkernels_amd`` imports it.
"""
from __future__ import annotations

import torch


def fix_paged_decode(kw: dict, cache_keys=("k_cache", "v_cache"),
                     generator: torch.Generator | None = None, page_dim: int = -2) -> None:
    """Make a paged decode's generically materialised inputs in range, in place, as
    the reference's bench does before timing a paged-decode candidate
    (``_fix_paged_decode``, fastkernels/bench.py:1305-1329).

    ``block_table`` gets page ids drawn uniformly from the cache's blocks (with
    repetition: sequences may share pages, and a page may recur within one), and
    ``cache_seqlens`` lengths uniform in [1, max_pages * page_size], so every length
    is addressable; ``max_seq_len`` (when present) becomes their maximum.  The
    caches keep their values (a zeroed cache would make the baseline output zeros).
    Geometry comes from the first cache: ``num_blocks`` from dim 0 and the page size
    from ``page_dim`` (-2, the reference's choice, fits the HND caches it fixes,
    ``[num_blocks, Hk, page_size, head_dim]``; pass 1 for NHD caches,
    ``[num_blocks, page_size, Hk, head_dim]``).  ``generator`` (a CPU generator)
    makes the draw reproducible; the tensors are moved to the cache's device."""
    caches = [kw.get(k) for k in cache_keys]
    bt, sl = kw.get("block_table"), kw.get("cache_seqlens")
    if not (all(isinstance(c, torch.Tensor) for c in caches)
            and isinstance(bt, torch.Tensor) and isinstance(sl, torch.Tensor)):
        raise ValueError("paged decode: missing cache/block_table/cache_seqlens")
    c0 = caches[0]
    num_blocks, page_size = int(c0.shape[0]), int(c0.shape[page_dim])
    max_pages = int(bt.shape[-1])
    kw["block_table"] = torch.randint(0, max(1, num_blocks), tuple(bt.shape), generator=generator,
                                      dtype=bt.dtype).to(c0.device)
    max_len = max(1, max_pages * page_size)
    lens = torch.randint(1, max_len + 1, tuple(sl.shape), generator=generator, dtype=sl.dtype)
    kw["cache_seqlens"] = lens.to(c0.device)
    if "max_seq_len" in kw:
        kw["max_seq_len"] = int(lens.max().item())
