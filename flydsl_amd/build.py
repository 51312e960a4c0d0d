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
# Kernels that must not use scratch: the MLA decode's inline-assembly DMA,
# waits and hazard cover were written for its register allocation without
# spills (a build whose extra code made it spill 36 VGPRs returned wrong
# rows).  The build reads the compiler's resource remarks for them and fails
# on any scratch.
NO_SCRATCH = {"mla_fp8.hip": ("mla_fp8_decode_kernel",)}
OUTPUT = os.path.join(HERE, "libpa_fp8.so")
# The checked build: the same kernels, which also record every index they
# clamp (pa_fp8_debug_violations in include/pa_fp8.h).
CHECKED_OUTPUT = os.path.join(HERE, "libpa_fp8_checked.so")
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _compile_cmd(src: str, obj: str, defines=()) -> list:
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
    if os.path.basename(src) in NO_SCRATCH:
        cmd += ["-Rpass-analysis=kernel-resource-usage"]
    return cmd + [f"-D{d}" for d in defines] + ["-c", src, "-o", obj]


def scratch_users(remarks: str, kernels) -> list:
    """(kernel symbol, bytes per lane) of each function in the compiler's
    kernel-resource-usage remarks whose name contains one of ``kernels`` and
    whose ScratchSize is not 0."""
    out, current = [], None
    for line in remarks.splitlines():
        if "Function Name:" in line:
            name = line.split("Function Name:", 1)[1].split()[0]
            current = name if any(k in name for k in kernels) else None
        elif current and "ScratchSize [bytes/lane]:" in line:
            n = int(line.split("ScratchSize [bytes/lane]:", 1)[1].split()[0])
            if n:
                out.append((current, n))
            current = None
    return out


def build_libraries(targets=((OUTPUT, ()), (CHECKED_OUTPUT, ("PA_FP8_CHECKED",))), verbose: bool = False) -> list:
    """Compile every HIP source for each (output, defines) target -- all
    compiles in parallel -- and link one shared library per target; returns
    their paths.

    Always recompiles.  Device code is built with packed-fp32 VALU ops
    disabled (the compiler would otherwise emit v_pk_{add,mul,fma}_f32).
    """
    noise = "is not a recognized feature for this target"
    jobs = []  # (output, objdir, objs, procs)
    for output, defines in targets:
        objdir = output + ".objs"
        os.makedirs(objdir, exist_ok=True)
        objs, procs = [], []
        for src in SOURCES:
            obj = os.path.join(objdir, os.path.basename(src) + ".o")
            cmd = _compile_cmd(src, obj, defines)
            if verbose:
                print(" ".join(cmd), flush=True)
            procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
            objs.append(obj)
        jobs.append((output, objdir, objs, procs))
    failed = []
    for output, _, _, procs in jobs:
        for src, p in procs:
            _, err = p.communicate()
            spills = scratch_users(err or "", NO_SCRATCH.get(os.path.basename(src), ()))
            err = "\n".join(l for l in (err or "").splitlines() if noise not in l and "remark:" not in l)
            if p.returncode != 0:
                failed.append(f"{os.path.basename(output)}: {os.path.basename(src)} ({p.returncode}):\n{err}")
            elif spills:
                failed.append(f"{os.path.basename(output)}: {os.path.basename(src)}: kernels that must not use scratch "
                              f"do: {spills}")
            elif verbose and err.strip():
                print(err, file=sys.stderr)
    if failed:
        raise RuntimeError("hipcc failed: " + "\n".join(failed))
    out = []
    for output, objdir, objs, _ in jobs:
        tmp = output + ".tmp"
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc link of {os.path.basename(output)} failed ({res.returncode}):\n{res.stderr}")
        os.replace(tmp, output)
        shutil.rmtree(objdir, ignore_errors=True)
        out.append(output)
    return out


def build_library(output: str = OUTPUT, verbose: bool = False) -> str:
    """The release library alone; returns its path."""
    return build_libraries(((output, ()),), verbose=verbose)[0]


if __name__ == "__main__":
    print("\n".join(build_libraries(verbose=True)))
