"""Build recipe for libmi355x_attn.so (gfx950 only).

Compiles every source under ``csrc/`` with ``hipcc --offload-arch=gfx950`` into
objects under ``csrc/_build/`` and links them into
``llm_infer_rust_amd/libmi355x_attn.so``. Run ``python -m llm_infer_rust_amd.build``.
Cross-compiles without a GPU.
"""
from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = CSRC / "_build"
LIB = PKG / "libmi355x_attn.so"
INCLUDE = PKG.parent / "include"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    "-fvisibility=hidden",
    f"-I{CSRC}",
    f"-I{INCLUDE}",
    # Keep the compiler from forming packed fp32 ops (v_pk_*_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # The direct-to-LDS copies set m0 in inline asm (declared clobbered).
    "-Wno-inline-asm",
]


def sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd = [HIPCC, *COMMON_FLAGS, "-x", "hip", "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")
    # hipcc's host pass warns that it does not know the packed-fp32 feature;
    # only surface other diagnostics.
    noise = "is not a recognized feature for this target"
    diag = [ln for ln in proc.stderr.splitlines() if ln.strip() and noise not in ln]
    if diag:
        sys.stderr.write("\n".join(diag) + "\n")
    return obj


def build(jobs: int | None = None) -> Path:
    """Compile all HIP sources and link the shared library. Always rebuilds."""
    BUILD.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(8, len(srcs))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
