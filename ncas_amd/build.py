"""Build `ncas_amd/libnca_hip.so` for gfx950 with hipcc (in-tree, no JIT cache)."""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
LIB = os.path.join(HERE, "libnca_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # keep hipcc from emitting packed-fp32 VALU ops (v_pk_*_f32) in any kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]
# per-source extra flags
SOURCES = {
    "nca_api.hip": [],
    # the streamed kernel keeps MFMA results and accumulators in VGPRs (its weight fragments are
    # pinned to AGPRs), so the VALU work on them needs no v_accvgpr copies
    "nca_stream.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "nca_stream32.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "nca_tiled.hip": [],
    # mlp_back32 keeps its weight fragments in AGPRs and its accumulators in VGPRs
    "nca_bptt.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "nca_prune.hip": [],
    "nca_metrics.hip": [],
    "nca_train.hip": [],
    "nca_boards.cpp": [],
}


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(
        line for line in (res.stdout + res.stderr).splitlines()
        if "packed-fp32-ops" not in line
    )
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{errs}")
    if verbose and errs.strip():
        print(errs, file=sys.stderr)


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile every HIP source (in parallel, `jobs` compilers at once) and link the shared
    library; always recompiles."""
    from concurrent.futures import ThreadPoolExecutor

    objs, cmds = [], []
    for src, extra in SOURCES.items():
        obj = os.path.join(CSRC, os.path.splitext(src)[0] + ".o")
        cmds.append([HIPCC, *FLAGS, *extra, "-I", INCLUDE, "-c", "-o", obj, os.path.join(CSRC, src)])
        objs.append(obj)
    jobs = jobs or min(len(cmds), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(jobs) as ex:
        for fut in [ex.submit(_run, cmd, verbose) for cmd in cmds]:
            fut.result()
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    for obj in objs:
        os.remove(obj)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
