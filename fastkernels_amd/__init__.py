"""fastkernels_amd — MI355X (gfx950) decode-step operators for the FastKernels serving path.

Hand-written HIP kernels behind a C ABI (``include/fastkernels_amd.h``), bound
with ctypes (``_native``), exposed as torch-facing ops (``ops``) and as drop-in
candidate classes with the reference's L1 operator names and signatures
(``candidate/L1/*.py``):

    RMSNorm, RotaryEmbedding, StoreKVCache, FlashAttnDecode, SiluAndMul

The candidate directory can be pointed at directly by the reference harness via
``FASTKERNELS_CANDIDATE_DIR=<repo>/fastkernels_amd/candidate``.
"""
from __future__ import annotations

from pathlib import Path

__version__ = "0.1.0"

CANDIDATE_DIR = Path(__file__).resolve().parent / "candidate"


def load() -> None:
    """Load libfk_amd.so now (raises if it has not been built)."""
    from . import _native

    _native.lib()
