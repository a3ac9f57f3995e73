"""Writes ``decode_step_configs.json``: a capture-format report of the benchmark
configurations C1-C5 (and the prefill / merge shapes) for the reference's own
harness, ``fastkernels bench`` (fastkernels/bench.py:274-300 loads every JSON under
``~/.fastkernels/captures``; the report layout is capture.py:187-238 and :497-526).

Each operator entry holds ``init`` variants (constructor arguments) and
``forward`` variants (argument shapes / dtypes keyed by parameter name, the
``**kwargs`` catch-all as a nested dict, strides only for non-contiguous views,
and ``init_variant_ids`` pairing each forward variant with its constructor).  The
harness materialises values itself (bench.py:787-870, with its paged-decode and
KV-store fix-ups, :1081-1096 and :1305-1330), so only shapes and dtypes are stored.

Run ``python -m fastkernels_amd.captures.make_reports`` to regenerate the file.
"""
from __future__ import annotations

import json
import math
from pathlib import Path

OUT = Path(__file__).resolve().parent / "decode_step_configs.json"
BASE = "fastkernels.tasks.baseline.L1."


def tensor(shape, dtype="bfloat16", stride=None):
    d = {"shape": list(shape), "dtype": dtype}
    if stride is not None:
        d["stride"] = list(stride)
    return d


def entry(inits, forwards):
    """inits: list of constructor-arg dicts; forwards: list of (init index, args, tag)."""
    return {
        "init": {"calls": len(inits), "variants": [{"count": 1, "args": a} for a in inits]},
        "forward": {"calls": len(forwards),
                    "variants": [{"count": 1, "args": a, "init_variant_ids": [i], "config": tag}
                                 for i, a, tag in forwards]},
    }


def build() -> dict:
    ops = {}
    ops[BASE + "rms_norm:RMSNorm"] = entry(
        [{"hidden_size": 1024, "eps": 1e-6, "elementwise_affine": True},
         {"hidden_size": 4096, "eps": 1e-6, "elementwise_affine": True}],
        [(0, {"x": tensor([256, 1024]), "residual": tensor([256, 1024])}, "C1"),
         (1, {"x": tensor([256, 4096]), "residual": tensor([256, 4096])}, "C4")])
    qkv_w = (32 + 2 * 8) * 128  # C4 q/k are row views of the fused qkv output
    ops[BASE + "rotary_emb:RotaryEmbedding"] = entry(
        [{"head_dim": 128, "max_position_embeddings": 40960, "rope_theta": 1000000.0,
          "rope_scaling_factor": 1.0, "rope_low_freq_factor": 1.0, "rope_high_freq_factor": 1.0,
          "rope_original_max_position_embeddings": None, "is_neox_style": True}],
        [(0, {"positions": tensor([256], "int64"),
              "query": tensor([256, 32 * 128], stride=[qkv_w, 1]),
              "key": tensor([256, 8 * 128], stride=[qkv_w, 1])}, "C4")])
    ops[BASE + "store_kvcache:StoreKVCache"] = entry(
        [{}],
        [(0, {"key": tensor([4096, 8, 128]), "value": tensor([4096, 8, 128]),
              "k_cache": tensor([2048, 256, 8, 128]), "v_cache": tensor([2048, 256, 8, 128]),
              "slot_mapping": tensor([4096], "int64")}, "C2"),
         (0, {"key": tensor([256, 8, 128], stride=[qkv_w, 128, 1]),
              "value": tensor([256, 8, 128], stride=[qkv_w, 128, 1]),
              "k_cache": tensor([4096, 256, 8, 128]), "v_cache": tensor([4096, 256, 8, 128]),
              "slot_mapping": tensor([256], "int64")}, "C4")])
    scale = 1.0 / math.sqrt(128)
    ops[BASE + "flash_attn_decode:FlashAttnDecode"] = entry(
        [{"num_heads": 32, "num_kv_heads": 8, "head_dim": 128, "page_size": 256},
         {"num_heads": 64, "num_kv_heads": 8, "head_dim": 128, "page_size": 256}],
        [(0, {"q": tensor([64, 32, 128]), "k_cache": tensor([4096, 256, 8, 128]),
              "v_cache": tensor([4096, 256, 8, 128]), "cache_seqlens": tensor([64], "int32"),
              "kwargs": {"block_table": tensor([64, 32], "int32"), "softmax_scale": scale,
                         "causal": True, "max_seq_len": 8192}}, "C3"),
         (0, {"q": tensor([256, 32, 128]), "k_cache": tensor([4096, 256, 8, 128]),
              "v_cache": tensor([4096, 256, 8, 128]), "cache_seqlens": tensor([256], "int32"),
              "kwargs": {"block_table": tensor([256, 16], "int32"), "softmax_scale": scale,
                         "causal": True, "max_seq_len": 4096}}, "C4"),
         (1, {"q": tensor([8, 64, 128]), "k_cache": tensor([4096, 256, 8, 128], "float8_e4m3fn"),
              "v_cache": tensor([4096, 256, 8, 128], "float8_e4m3fn"),
              "cache_seqlens": tensor([8], "int32"),
              "kwargs": {"block_table": tensor([8, 512], "int32"), "softmax_scale": scale,
                         "causal": True, "max_seq_len": 131072}}, "C5")])
    ops[BASE + "silu_and_mul:SiluAndMul"] = entry(
        [{}], [(0, {"x": tensor([256, 2 * 12288])}, "C4")])
    ops[BASE + "flash_attn_prefill:FlashAttnPrefill"] = entry(
        [{"num_heads": 32, "num_kv_heads": 8, "head_dim": 128}],
        [(0, {"q": tensor([2048, 32, 128]), "k": tensor([8, 256, 8, 128]),
              "v": tensor([8, 256, 8, 128]), "cu_seqlens_q": tensor([2], "int32"),
              "cu_seqlens_k": tensor([2], "int32"), "max_seqlen_q": 2048, "max_seqlen_k": 2048,
              "kwargs": {"softmax_scale": scale, "causal": True,
                         "block_table": tensor([1, 8], "int32")}}, "prefill 1x2048")])
    ops[BASE + "merge_attn_states:MergeAttnStates"] = entry(
        [{}],
        [(0, {"output": tensor([8192, 32, 128]), "prefix_output": tensor([8192, 32, 128]),
              "prefix_lse": tensor([32, 8192], "float32"),
              "suffix_output": tensor([8192, 32, 128]),
              "suffix_lse": tensor([32, 8192], "float32"),
              "output_lse": tensor([32, 8192], "float32")}, "merge")])
    return {"scenario": "fastkernels_amd decode-step configurations C1-C5 (synthetic)",
            "operators": ops}


def main() -> None:
    OUT.write_text(json.dumps(build(), indent=1) + "\n")
    print(OUT)


if __name__ == "__main__":
    main()
