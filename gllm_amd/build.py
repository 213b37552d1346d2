"""Builds libgllm_attn.so (gfx950) in-tree with hipcc.

    python -m gllm_amd.build                # or gllm_amd.build.build()

Each .hip unit is compiled to an object in parallel, then linked into
``gllm_amd/lib/libgllm_attn.so``.  Units whose arithmetic must round like the
reference's torch ops are compiled with ``-ffp-contract=off``.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libgllm_attn.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

SOURCES = ["paged_attention.hip", "paged_attention_f16.hip", "api.hip", "rope_kv_write.hip", "attention_f32.hip",
           "metadata.hip", "qkv_proj.hip"]
NO_CONTRACT = {"rope_kv_write.hip", "attention_f32.hip", "qkv_proj.hip"}
# MFMA accumulators stay in VGPRs (no per-tile AGPR<->VGPR copies)
EXTRA = {"paged_attention.hip": ["-mllvm", "--amdgpu-mfma-vgpr-form"],
         "paged_attention_f16.hip": ["-mllvm", "--amdgpu-mfma-vgpr-form"]}
COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # packed fp32 VALU ops are disabled on purpose for every HIP unit
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _compile(src: str) -> str:
    obj = os.path.join(LIBDIR, src.replace(".hip", ".o"))
    cmd = [HIPCC, *COMMON, "-c", os.path.join(CSRC, src), "-o", obj]
    if src in NO_CONTRACT:
        cmd.insert(1, "-ffp-contract=off")
    cmd[1:1] = EXTRA.get(src, [])
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr[-4000:]}")
    return obj


def _link(objs, out, extra):
    tmp = out + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, *extra]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, out)
    for o in objs:
        os.remove(o)


def build(verbose: bool = False) -> str:
    os.makedirs(LIBDIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    # roctx ranges around the entry points
    _link(objs, LIB, ["-L/opt/rocm/lib", "-lrocprofiler-sdk-roctx", "-Wl,-rpath,/opt/rocm/lib"])
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
