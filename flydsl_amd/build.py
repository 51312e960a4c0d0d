"""Build ``libpa_fp8.so`` in-tree with hipcc for gfx950 (no GPU needed)."""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
SOURCES = [os.path.join(CSRC, n) for n in ("pa_fp8.hip", "rope_cache.hip", "qk_norm_rope.hip")]
OUTPUT = os.path.join(HERE, "libpa_fp8.so")
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def build_library(output: str = OUTPUT, verbose: bool = False) -> str:
    """Compile every HIP source into one shared library; returns its path.

    Always recompiles.  Device code is built with packed-fp32 VALU ops
    disabled (the compiler would otherwise emit v_pk_{add,mul,fma}_f32).
    """
    tmp = output + ".tmp"
    cmd = [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-Wall",
        f"-I{INCLUDE}",
        f"-I{CSRC}",
        "-Xclang",
        "-target-feature",
        "-Xclang",
        "-packed-fp32-ops",
        # MFMA accumulators in VGPRs: the online-softmax rescale and the
        # slot merges are VALU work on them (no AGPR round trips).
        "-mllvm",
        "-amdgpu-mfma-vgpr-form",
        *SOURCES,
        "-o",
        tmp,
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (res.stderr or "").splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, output)
    return output


if __name__ == "__main__":
    print(build_library(verbose=True))
