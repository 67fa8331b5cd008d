"""Builds libk44wavec.so (gfx950) next to this file with hipcc.

Usage: python -m snntome_amd.build   (also called by __graft_entry__.build()).
"""
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = HERE / "libk44wavec.so"
ARCH = os.environ.get("K44_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Wno-unused-result",
    # Packed fp32 (v_pk_*_f32) code generation stays off on this pool.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{CSRC}",
    f"-I{HERE.parent / 'include'}",
]


def build(verbose: bool = True) -> Path:
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, *HIPCC_FLAGS, str(CSRC / "k44_wave_executor.hip"), "-o", str(tmp)]
    if verbose:
        print("[build]", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "packed-fp32-ops"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        sys.stderr.write(err + "\n")
        raise RuntimeError(f"hipcc failed ({res.returncode}) building {LIB.name}")
    if verbose and err.strip():
        sys.stderr.write(err + "\n")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build()
