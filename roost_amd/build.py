"""Builds libroost_kernels_gfx950.so in-tree with hipcc (gfx950 only).

The library is the product: the C ABI of include/roost_kernels.h and include/roost_amd.h. It is compiled from
roost_amd/csrc with explicit hipcc invocations (no JIT, no torch extension), one object per source, linked into one
shared object next to this file so that it travels with the source tree.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB_NAME = "libroost_kernels_gfx950.so"
LIB_PATH = HERE / LIB_NAME
SOURCES = ["registry.cpp", "cache_write.hip", "paged_attention.hip", "gated_delta_rule.hip", "gdn_layer.hip", "qk_rope.hip", "plan_region.hip"]

# Packed-FP32 instructions are kept out of every HIP object (the compiler would otherwise form v_pk_* from scalar
# float code); the host pass of hipcc warns that it does not know the feature, which is harmless.
HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950", "-munsafe-fp-atomics",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fvisibility=hidden", "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the gfx950 library cannot be built")
    return path


# Per-source code-generation options. The GDN scan keeps its MFMA accumulators in architectural VGPRs (its
# compute wavefronts read them with VALU every chunk; the AGPR form costs a copy per read).
SOURCE_FLAGS = {"gated_delta_rule.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def _compile(src: str) -> Path:
    obj = BUILD / (Path(src).stem + ".o")
    lang = ["-x", "hip"] if src.endswith(".cpp") else []
    cmd = [hipcc(), *HIPCC_FLAGS, *SOURCE_FLAGS.get(src, []), *lang, "-I", str(ROOT / "include"), "-c", str(CSRC / src),
           "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{res.stderr}")
    warnings = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if warnings:
        print("\n".join(warnings), file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    """Compiles every source and links the library; returns its path."""
    BUILD.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(4, os.cpu_count() or 1)) as pool:
        objs = list(pool.map(_compile, SOURCES))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), "-shared", "-fPIC", "--offload-arch=gfx950", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    # The name Roost's loader derives for arch id 950 (libroost_kernels_sm<N>.so), pointing at the same file.
    alias = HERE / "libroost_kernels_sm950.so"
    if alias.is_symlink() or alias.exists():
        alias.unlink()
    alias.symlink_to(LIB_NAME)
    # The gfx950 manifest entries (variants, flags, constraints, the file's size and digest) follow every build.
    from . import manifest
    from . import KernelLibrary

    manifest.write(KernelLibrary(LIB_PATH), LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} and {manifest.MANIFEST_PATH.name}")
    return LIB_PATH


if __name__ == "__main__":
    build()
