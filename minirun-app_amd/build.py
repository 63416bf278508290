"""Builds the gfx950 libraries in-tree with hipcc.

    python minirun-app_amd/build.py          # libminirun_hip.so + libminirun_selftest.so

Outputs go to minirun-app_amd/lib/.  Every HIP source is compiled for gfx950
only, with packed-fp32 instruction selection disabled.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "lib")
OBJ = os.path.join(HERE, "lib", "obj")
ROOT = os.path.dirname(HERE)

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
    "-I", CSRC,
]

LIB_SOURCES = ["capi.cpp", "capi_adopt.cpp", "capi_block.cpp", "capi_prefill.cpp", "capi_topk.cpp", "decode.hip", "affine.hip",
               "mla_block.hip", "prefill.hip", "topk.hip", "indexer.hip", "linear.hip", "gemm.hip", "generic.hip"]
# Per-source flags.  The decode kernel keeps its MFMA accumulators in VGPRs
# (VGPR-form MFMA): with the AGPR form the compiler shuttles all 64 of them
# through v_accvgpr moves on every 32-row step.
EXTRA = {"decode.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}
SELFTEST_SOURCES = ["selftest.hip"]


def _compile(src: str) -> str:
    out = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, *EXTRA.get(src, []), "-c", os.path.join(CSRC, src), "-o", out]
    if src.endswith(".cpp"):
        cmd.insert(1, "-x")
        cmd.insert(2, "hip")
    r = subprocess.run(cmd, capture_output=True, text=True)
    msg = "\n".join(line for line in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in line)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{msg}")
    if msg.strip():
        print(msg, file=sys.stderr)
    return out


def _link(objs, name):
    out = os.path.join(LIB, name)
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", out + ".tmp"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed for {name}:\n{r.stdout}{r.stderr}")
    os.replace(out + ".tmp", out)
    return out


def build(jobs: int = 8) -> list[str]:
    os.makedirs(OBJ, exist_ok=True)
    srcs = LIB_SOURCES + SELFTEST_SOURCES
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(srcs)))) as ex:
        objs = dict(zip(srcs, ex.map(_compile, srcs)))
    return [
        _link([objs[s] for s in LIB_SOURCES], "libminirun_hip.so"),
        _link([objs[s] for s in SELFTEST_SOURCES], "libminirun_selftest.so"),
    ]


if __name__ == "__main__":
    for p in build():
        print(p)
