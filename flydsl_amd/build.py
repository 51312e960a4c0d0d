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
SOURCES = [os.path.join(CSRC, n) for n in ("pa_fp8.hip", "rope_cache.hip", "qk_norm_rope.hip", "mla_fp8.hip")]
# MFMA results in VGPRs: the online-softmax rescale and the slot merges of
# the paged-attention kernels are VALU work on them (no AGPR round trips),
# and the MLA kernel keeps its logits there while its value accumulators are
# pinned to AGPRs by inline assembly.
VGPR_FORM = {"pa_fp8.hip", "rope_cache.hip", "qk_norm_rope.hip", "mla_fp8.hip"}
OUTPUT = os.path.join(HERE, "libpa_fp8.so")
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _compile_cmd(src: str, obj: str) -> list:
    cmd = [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-Wall",
        f"-I{INCLUDE}",
        f"-I{CSRC}",
        "-Xclang",
        "-target-feature",
        "-Xclang",
        "-packed-fp32-ops",
    ]
    if os.path.basename(src) in VGPR_FORM:
        cmd += ["-mllvm", "-amdgpu-mfma-vgpr-form"]
    return cmd + ["-c", src, "-o", obj]


def build_library(output: str = OUTPUT, verbose: bool = False) -> str:
    """Compile every HIP source (in parallel) and link one shared library;
    returns its path.

    Always recompiles.  Device code is built with packed-fp32 VALU ops
    disabled (the compiler would otherwise emit v_pk_{add,mul,fma}_f32).
    """
    noise = "is not a recognized feature for this target"
    objdir = output + ".objs"
    os.makedirs(objdir, exist_ok=True)
    objs, procs = [], []
    for src in SOURCES:
        obj = os.path.join(objdir, os.path.basename(src) + ".o")
        cmd = _compile_cmd(src, obj)
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
        objs.append(obj)
    failed = []
    for src, p in procs:
        _, err = p.communicate()
        err = "\n".join(l for l in (err or "").splitlines() if noise not in l)
        if p.returncode != 0:
            failed.append(f"{os.path.basename(src)} ({p.returncode}):\n{err}")
        elif verbose and err.strip():
            print(err, file=sys.stderr)
    if failed:
        raise RuntimeError("hipcc failed: " + "\n".join(failed))
    tmp = output + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc link failed ({res.returncode}):\n{res.stderr}")
    os.replace(tmp, output)
    shutil.rmtree(objdir, ignore_errors=True)
    return output


if __name__ == "__main__":
    print(build_library(verbose=True))
