"""Per-workgroup timeline of one paged-attention launch on the GPU.

    python -m gllm_amd.build --timestamps        # libgllm_attn_ts.so
    python -m gllm_amd.timeline --config d       # b, c, d or e; --split N (0 auto, -1 page-balanced)

Loads the timestamp build of the library (the kernels record every
workgroup's start and end with the 100 MHz ``s_memrealtime`` counter, its
kind, XCD and keys), runs the benchmark configuration's launch a few times
over rotating KV pools (``--copies``, as bench.py) and prints, for the last
launch: the span from the first start to the last
end, the start spread, durations and end times by kind, the end time of each
XCD, and how many workgroups of each kind are running every 25 µs.  The
launch is timed with HIP events too, so the time outside the workgroups'
span (dispatch and drain) shows.
"""
from __future__ import annotations

import argparse
import ctypes
import os

import numpy as np
import torch

from gllm_amd import _lib, build, workloads

KINDS = {0: "decode item", 1: "prefill item", 2: "decode segments"}


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--config", default="d", choices=["b", "c", "d", "e"])
    ap.add_argument("--split", type=int, default=0, help="split_tokens of the plan (0: the planner's choice)")
    ap.add_argument("--reps", type=int, default=5)
    ap.add_argument("--save", default="", help="also write the raw records (int64 [n, 4]) to this .npy file")
    ap.add_argument("--copies", type=int, default=4,
                    help="KV pools the launches rotate through (as bench.py), so a batch smaller than the "
                         "256 MB Infinity Cache is still read from HBM")
    args = ap.parse_args()
    if not os.path.exists(build.TS_LIB):
        raise SystemExit(f"{build.TS_LIB} not found: run `python -m gllm_amd.build --timestamps` first")
    lib = _lib.load(build.TS_LIB)
    lib.gllm_debug_timestamps.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    lib.gllm_debug_timestamps.restype = ctypes.c_int
    from gllm_amd import paged   # after the timestamp library is the loaded one

    dev = torch.device("cuda", 0)
    b = getattr(workloads, f"config_{args.config}")()
    xs = []
    for i in range(max(1, args.copies)):
        c = workloads.PagedBatch(**{k: getattr(b, k) for k in (
            "name", "ctx_lens", "q_lens", "num_q_heads", "num_kv_heads", "head_dim", "block_size",
            "num_blocks", "dtype", "rope_theta", "kv_dtype")})
        xs.append(workloads.materialize(c, dev, values_on_device=True, seed=2 + i))
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=b.num_q_heads, num_kv_heads=b.num_kv_heads,
                               head_dim=b.head_dim, block_size=b.block_size, dtype=b.dtype, device=dev,
                               split_tokens=args.split)
    out = torch.empty_like(xs[0].q)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for r in range(max(1, args.reps)):
        x = xs[r % len(xs)]
        rope = (x.cos, x.sin, "position") if args.config == "c" else None
        e0.record()
        paged.paged_attention(plan, x.q, x.k_cache, x.v_cache, x.block_table, out=out, rope=rope)
        e1.record()
        torch.cuda.synchronize()
    n = min(plan.info["work_items"], 1 << 15)
    buf = np.zeros(4 * n, dtype=np.int64)
    rc = lib.gllm_debug_timestamps(buf.ctypes.data, buf.nbytes)
    if rc:
        raise RuntimeError(f"gllm_debug_timestamps: hip error {rc}")
    d = buf.reshape(n, 4)
    if args.save:
        np.save(args.save, d)
    t0 = d[:, 0].min()
    st, en = (d[:, 0] - t0) / 100.0, (d[:, 1] - t0) / 100.0      # µs
    kind, xcd, keys = d[:, 2] & 0xff, (d[:, 2] >> 8) & 15, d[:, 3]
    dur = en - st
    print(f"config ({args.config}) {b.name}: plan {plan.info}")
    print(f"launch {e0.elapsed_time(e1) * 1e3:.1f} µs (HIP events); workgroups {n}: span {en.max():.1f} µs, "
          f"starts within {np.sort(st)[min(n - 1, 255)]:.1f} µs for the first 256")
    for k, name in KINDS.items():
        m = kind == k
        if m.any():
            print(f"  {name:16s} n {m.sum():5d}  duration mean {dur[m].mean():7.1f} max {dur[m].max():7.1f} µs  "
                  f"end mean {en[m].mean():7.1f} max {en[m].max():7.1f}  keys mean {keys[m].mean():8.0f}")
    print("  end per XCD:", " ".join(f"{en[xcd == c].max():.1f}" for c in range(8) if (xcd == c).any()))
    print("  end percentiles 10/50/90/100:", " ".join(f"{np.percentile(en, q):.1f}" for q in (10, 50, 90, 100)))
    for t in np.arange(0.0, en.max(), 25.0):
        run = (st <= t) & (en > t)
        parts = [f"{KINDS[k]} {int((run & (kind == k)).sum())}" for k in KINDS if (kind == k).any()]
        print(f"  t={t:7.1f} µs running: " + ", ".join(parts))


if __name__ == "__main__":
    main()
