"""Builds libramvamp_attn.so in-tree with hipcc for gfx950.

    python -m ramvamp_amd.build

Every HIP source is compiled for gfx950 only, with packed-FP32 instruction
selection disabled (-Xclang -target-feature -Xclang -packed-fp32-ops: the
compiler would otherwise form v_pk_*_f32 from plain float code). hipcc's host
pass warns that it does not know the feature; that warning is expected.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libramvamp_attn.so")
SOURCES = ["rv_abi.cpp", "rv_prologue.hip", "rv_decode.hip", "rv_prefill.hip", "rv_quant.hip", "rv_gemv_abi.cpp",
           "rv_block_abi.cpp", "rv_router.hip", "rv_floors.hip"]
# Per-source extra flags. The prefill kernels hold MFMA accumulators and
# their softmax operands together; the default heuristic places the
# accumulators in AGPRs and copies them through VGPRs every tile, so their
# MFMAs are forced to the VGPR form.
EXTRA = {"rv_prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
NOISE = "is not a recognized feature for this target"


def _run(cmd: list[str]) -> list[str]:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    msgs = [ln for ln in (proc.stdout + proc.stderr).splitlines() if NOISE not in ln]
    if proc.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + " ".join(cmd) + "\n" + "\n".join(msgs))
    return msgs


def build(verbose: bool = False) -> str:
    """Compile every source to an object (in parallel), then link the library."""
    objdir = os.path.join(HERE, "_obj")
    os.makedirs(objdir, exist_ok=True)
    objs, cmds = [], []
    for src in SOURCES:
        obj = os.path.join(objdir, src + ".o")
        objs.append(obj)
        cmds.append([HIPCC, *FLAGS, *EXTRA.get(src, []), "-c", "-o", obj, os.path.join(CSRC, src)])
    with ThreadPoolExecutor(max_workers=len(cmds)) as pool:
        msgs = [m for ms in pool.map(_run, cmds) for m in ms]
    tmp = OUT + ".tmp"
    msgs += _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    if verbose and msgs:
        print("\n".join(msgs), file=sys.stderr)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
