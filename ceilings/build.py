"""Build recipe for the measurement-only ceilings library (bench.py's "ceilings" section).

Compiles ``ceilings/ceilings.hip`` for gfx950 into ``ceilings/libmi355x_calib.so`` with the
product library's compiler flags. No product path loads it. Run
``python -m ceilings.build`` from the repository root (``__graft_entry__.build()`` runs it).
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "ceilings.hip"
LIB = HERE / "libmi355x_calib.so"

sys.path.insert(0, str(HERE.parent))
from llm_infer_rust_amd.build import COMMON_FLAGS, HIPCC  # noqa: E402


def build() -> Path:
    """Compile the ceilings library. Always rebuilds."""
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, *COMMON_FLAGS, "-shared", str(SRC), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {SRC.name}:\n{proc.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
