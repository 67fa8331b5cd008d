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
    # Leading scalar and pointer kernel arguments arrive preloaded in SGPRs (gfx950 kernarg
    # preload), so a kernel's first dependent load does not wait for a kernarg-segment read.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    f"-I{CSRC}",
    f"-I{HERE.parent / 'include'}",
]


SOURCES = ["k44_wave_executor.hip", "k44_exec_build.hip", "k44_exec_schedule.hip", "k44_exec_launch.hip", "kernels/k44_valu.hip", "kernels/k44_aux.hip", "kernels/k44_mfma_dispatch.hip",
           "kernels/k44_mfma_nt16.hip", "kernels/k44_mfma_nt32.hip", "kernels/k44_mfma_nt64.hip",
           "kernels/k44_mfma_nt128.hip", "kernels/k44_mfma_narrow.hip", "kernels/k44_mfma_dma.hip", "kernels/k44_token64.hip",
           "kernels/k44_spatial.hip", "kernels/k44_program.hip"]
BUILD_DIR = HERE / "_build"


def _clean(stderr: str) -> str:
    return "\n".join(l for l in stderr.splitlines() if "packed-fp32-ops" not in l)


def _stale(obj: Path, src: Path) -> bool:
    """The object is older than its source or than any header of the tree."""
    if not obj.exists():
        return True
    t = obj.stat().st_mtime
    heads = [*CSRC.rglob("*.hpp"), *(HERE.parent / "include").glob("*.h")]
    return any(f.stat().st_mtime > t for f in [src, *heads])


def build(verbose: bool = True, changed_only: bool = False) -> Path:
    """Compiles every translation unit for gfx950 (in parallel) and links libk44wavec.so.
    changed_only: recompile only objects older than their source or a header."""
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    BUILD_DIR.mkdir(exist_ok=True)
    objs, procs = [], []
    for src in SOURCES:
        obj = BUILD_DIR / (Path(src).stem + ".o")
        if changed_only and not _stale(obj, CSRC / src):
            objs.append(obj)
            continue
        cmd = [hipcc, *[f for f in HIPCC_FLAGS if f != "-shared"], "-c", str(CSRC / src),
               "-o", str(obj)]
        if verbose:
            print("[build]", " ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                                            text=True)))
        objs.append(obj)
    failed = []
    for src, p in procs:
        _, err = p.communicate()
        err = _clean(err)
        if p.returncode != 0:
            failed.append(src)
            sys.stderr.write(err + "\n")
        elif verbose and err.strip():
            sys.stderr.write(err + "\n")
    if failed:
        raise RuntimeError(f"hipcc failed on {failed}")
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print("[build]", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(_clean(res.stderr) + "\n")
        raise RuntimeError(f"hipcc link failed ({res.returncode}) for {LIB.name}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build(changed_only="--changed" in sys.argv)
