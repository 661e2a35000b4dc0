"""Build ``libmetile_amd.so`` in-tree with hipcc for gfx950.

Usage: ``python -m metile_amd.build`` (or ``metile_amd.build.build()``). Every call compiles
all sources; objects go to ``metile_amd/_build/`` and the shared library to
``metile_amd/libmetile_amd.so`` (both git-ignored).
"""

from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
BUILD = PKG / "_build"
LIB = PKG / "libmetile_amd.so"
ARCH = "gfx950"

# -packed-fp32-ops keeps the compiler from forming packed fp32 VALU instructions.
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


# Per-source extra flags. The ring GEMM and the column-block kernel keep their MFMA results in
# ordinary VGPRs (the VALU fix-up reads every one; in accumulation registers each read costs a
# copy).
FILE_FLAGS = {"affine_gemm_ring.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
              "affine_qmv_block.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build metile_amd)")


def sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def source_digest() -> str:
    """SHA-256 over the compiler flags and every kernel, boundary and header source, in name
    order: the library reports it (``mt_source_digest``) so that persistent tuning decisions
    are keyed to the code they were measured on."""
    h = hashlib.sha256(" ".join(HIP_FLAGS).encode())
    for name in sorted(FILE_FLAGS):
        h.update((name + " " + " ".join(FILE_FLAGS[name])).encode())
    for path in sorted([*sources(), *CSRC.glob("*.h"), *INCLUDE.glob("*.h")],
                       key=lambda p: p.name):
        h.update(path.name.encode() + b"\0" + path.read_bytes() + b"\0")
    return h.hexdigest()


def _compile(src: Path, digest: str) -> Path:
    obj = BUILD / (src.name + ".o")
    cmd = [hipcc(), *HIP_FLAGS, *FILE_FLAGS.get(src.name, []), f"-DMT_SOURCE_DIGEST=\"{digest}\"",
           f"-I{CSRC}", f"-I{INCLUDE}",
           "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every HIP/C++ source and link ``libmetile_amd.so``; returns its path."""
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    digest = source_digest()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as pool:
        objs = list(pool.map(lambda src: _compile(src, digest), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
