"""Build libpolyattn.so (the HIP kernels + C ABI) in-tree with hipcc for gfx950.

Usage: ``python -m poly_attention._build`` (with ``poly-attention_amd`` on ``sys.path``) or
``poly_attention._build.build()``.  The library lands in ``poly_attention/_lib/`` so that it
travels with the source tree; object files go to ``<repo>/_build/`` (git-ignored).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
SRC_DIR = PKG_DIR.parent / "csrc"
REPO_ROOT = PKG_DIR.parent.parent
INCLUDE_DIR = REPO_ROOT / "include"
BUILD_DIR = REPO_ROOT / "_build"
LIB_DIR = PKG_DIR / "_lib"
LIB_NAME = "libpolyattn.so"

ARCH = "gfx950"

# -packed-fp32-ops: never emit v_pk_{add,mul,fma}_f32 (unreliable on this pool's parts).
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
    f"-I{INCLUDE_DIR}",
    f"-I{SRC_DIR}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain (ROCm) is required to build libpolyattn")


def sources() -> list[Path]:
    return sorted(SRC_DIR.glob("*.hip"))


def _compile(src: Path, extra: list[str]) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass does not know the packed-fp32 target feature; that warning is harmless
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = True, extra_flags: list[str] | None = None) -> Path:
    """Compile every csrc/*.hip for gfx950 and link libpolyattn.so; returns its path."""
    extra = list(extra_flags or [])
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    if verbose:
        print(f"[polyattn] compiling {len(srcs)} sources for {ARCH}", flush=True)
    workers = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", "8"))))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(lambda s: _compile(s, extra), srcs))
    out = LIB_DIR / LIB_NAME
    tmp = LIB_DIR / (LIB_NAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{proc.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"[polyattn] built {out}", flush=True)
    return out


if __name__ == "__main__":
    build()
