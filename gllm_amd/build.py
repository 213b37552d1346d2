"""Builds libgllm_attn.so (gfx950) in-tree with hipcc.

    python -m gllm_amd.build                # or gllm_amd.build.build()
    python -m gllm_amd.build --timestamps   # libgllm_attn_ts.so, for gllm_amd.timeline

Each .hip unit is compiled to an object in parallel, then linked into
``gllm_amd/lib/libgllm_attn.so`` (the memory-path probes of bench.py's box
ceilings into ``gllm_amd/lib/libgllm_probe.so``).  Units whose arithmetic must round like the
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

SOURCES = ["api.hip", "rope_kv_write.hip", "paged_attention.hip", "attention_f32.hip", "metadata.hip",
           "qkv_proj.hip"]
# memory-path probes behind bench.py's box ceilings (own library, not the attention path)
PROBE_SOURCES = ["probe.hip"]
PROBE_LIB = os.path.join(LIBDIR, "libgllm_probe.so")
NO_CONTRACT = {"rope_kv_write.hip", "attention_f32.hip", "qkv_proj.hip"}
# MFMA accumulators stay in VGPRs (no per-tile AGPR<->VGPR copies)
EXTRA = {"paged_attention.hip": ["-mllvm", "--amdgpu-mfma-vgpr-form"]}
COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # packed fp32 VALU ops are disabled on purpose for every HIP unit
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


TS_LIB = os.path.join(LIBDIR, "libgllm_attn_ts.so")   # per-workgroup timestamp build (gllm_amd.timeline)


def _compile(src: str, defines=()) -> str:
    obj = os.path.join(LIBDIR, src.replace(".hip", "_ts.o" if defines else ".o"))
    cmd = [HIPCC, *COMMON, *[f"-D{d}" for d in defines], "-c", os.path.join(CSRC, src), "-o", obj]
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
    with ThreadPoolExecutor(max_workers=min(4, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(_compile, SOURCES + PROBE_SOURCES))
    # roctx ranges around the entry points
    _link(objs[:len(SOURCES)], LIB, ["-L/opt/rocm/lib", "-lrocprofiler-sdk-roctx", "-Wl,-rpath,/opt/rocm/lib"])
    _link(objs[len(SOURCES):], PROBE_LIB, [])
    if verbose:
        print(f"built {LIB} and {PROBE_LIB}")
    return LIB


def build_timestamps(verbose: bool = False) -> str:
    """The attention library with per-workgroup timestamps
    (-DGLLM_TIMESTAMPS) as libgllm_attn_ts.so, for ``gllm_amd.timeline``."""
    os.makedirs(LIBDIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(4, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(lambda src: _compile(src, ("GLLM_TIMESTAMPS",)), SOURCES))
    _link(objs, TS_LIB, ["-L/opt/rocm/lib", "-lrocprofiler-sdk-roctx", "-Wl,-rpath,/opt/rocm/lib"])
    if verbose:
        print(f"built {TS_LIB}")
    return TS_LIB


if __name__ == "__main__":
    if "--timestamps" in sys.argv[1:]:
        build_timestamps(verbose=True)
    else:
        build(verbose=True)
    sys.exit(0)
