"""Build recipe for libfk_amd.so, the gfx950 C-ABI library.

Each ``csrc/*.hip`` file is compiled by ``hipcc --offload-arch=gfx950`` in
parallel, then linked into ``fastkernels_amd/_lib/libfk_amd.so`` (in-tree, so a
snapshot of the repository carries it to a GPU host).  The build always
recompiles: it is the "does it build" check as well as the build.

Usage: ``python -m fastkernels_amd.build`` (or ``__graft_entry__.build()``).
``python -m fastkernels_amd.build --define NAME --out DIR`` builds a variant
library with extra preprocessor definitions into DIR/libfk_amd.so instead (the
A/B tile forms of fk_paged_decode.hip); load it with FASTKERNELS_AMD_LIB.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_DIR = PKG_DIR / "_lib"
LIB_PATH = LIB_DIR / "libfk_amd.so"
OBJ_DIR = PKG_DIR / "_build"
ARCH = "gfx950"

# Packed-FP32 VALU ops are disabled in all device code (hipcc still forms
# ordinary FMAs); the host pass ignores the feature with a warning.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


def _compile(src: Path, obj_dir: Path = OBJ_DIR, defines: tuple = (), cflags: tuple = ()) -> Path:
    obj = obj_dir / (src.stem + ".o")
    cmd = [_hipcc(), *HIP_FLAGS, *cflags, *(f"-D{d}" for d in defines), "-c", str(src), "-o",
           str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")
    return obj


def build(verbose: bool = True, defines: tuple = (), out_dir: Path | None = None,
          cflags: tuple = ()) -> Path:
    """Compile every csrc/*.hip for gfx950 and link libfk_amd.so; return its path.
    With out_dir, objects and library go there (a variant build with `defines`
    and extra compiler flags `cflags`)."""
    obj_dir = OBJ_DIR if out_dir is None else Path(out_dir) / "_obj"
    lib_path = LIB_PATH if out_dir is None else Path(out_dir) / "libfk_amd.so"
    obj_dir.mkdir(parents=True, exist_ok=True)
    lib_path.parent.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(sources), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(lambda src: _compile(src, obj_dir, tuple(defines), tuple(cflags)),
                           sources))
    tmp = lib_path.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, lib_path)
    if verbose:
        extra = f" with {', '.join(defines)}" if defines else ""
        print(f"built {lib_path} from {len(sources)} sources{extra}", file=sys.stderr)
    return lib_path


if __name__ == "__main__":
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--define", action="append", default=[], help="preprocessor macro (repeatable)")
    ap.add_argument("--cflag", action="append", default=[], help="extra hipcc flag (repeatable)")
    ap.add_argument("--out", type=Path, default=None, help="output directory of a variant build")
    a = ap.parse_args()
    if (a.define or a.cflag) and a.out is None:
        ap.error("--define / --cflag need --out (the in-tree library is always the default build)")
    build(defines=tuple(a.define), out_dir=a.out, cflags=tuple(a.cflag))
