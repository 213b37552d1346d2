"""Benchmark of the gLLM attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs b,c,d,e]

Prints ONE JSON line.  The headline (``value``) is BASELINE config (b): decode
paged attention at the Llama-3.2-1B head shape, in GB/s of compulsory HBM
bytes per launch, inputs resident in HBM, KV pools rotated so the 256 MB
Infinity Cache cannot serve them (cold HBM).  A "step" is one attention launch
over the whole batch (one layer's attention).  Configs (c)-(e) are reported
in ``extra`` with their own roofline figures; (c)'s step also includes the
fused RoPE + KV write kernel.  The CPU baseline times the reference's path
(padded gather, GQA expand, dense softmax attention, fp32 torch) on the
host's cores for config (b).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from gllm_amd import paged, workloads  # noqa: E402

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def _events_time(launches, warmup, steps):
    """Run ``launches[i % len]`` warmup + steps times on the current stream;
    returns (per-launch ms list, wall ms per step) from HIP events."""
    for i in range(warmup):
        launches[i % len(launches)]()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(steps):
        starts[i].record()
        launches[i % len(launches)]()
        ends[i].record()
    t1.record()
    torch.cuda.synchronize()
    per = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    return per, t0.elapsed_time(t1) / steps


def _graph_time(launches, warmup, steps):
    """Capture ``steps`` launches (``launches[i % len]``) in one HIP graph,
    the way a serving loop runs its decode steps, replay it once (or more)
    to warm up, then time exactly one replay = ``steps`` steps, bracketed by
    synchronisations; returns ms per step."""
    cur = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    side.wait_stream(cur)
    with torch.cuda.stream(side):              # warm-up outside capture
        for f in launches:
            f()
    cur.wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            launches[i % len(launches)]()
    for _ in range(max(1, -(-warmup // steps))):
        g.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    g.replay()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps


def _copies(b: workloads.PagedBatch, n: int, dev, on_device: bool):
    """n independent pools (same lengths, own values and tables) so repeated
    launches stream HBM rather than the Infinity Cache."""
    out = []
    for i in range(n):
        c = workloads.PagedBatch(**{k: getattr(b, k) for k in (
            "name", "ctx_lens", "q_lens", "num_q_heads", "num_kv_heads", "head_dim", "block_size",
            "num_blocks", "dtype", "rope_theta", "kv_dtype")})
        out.append(workloads.materialize(c, dev, values_on_device=on_device, seed=2 + i))
    return out


def bench_decode(b, copies, warmup, steps, split, dev, hw=0):
    bs = _copies(b, copies, dev, on_device=True)
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=b.num_q_heads, num_kv_heads=b.num_kv_heads,
                               head_dim=b.head_dim, block_size=b.block_size, dtype=b.dtype, device=dev,
                               split_tokens=split, heads_per_wg=hw)
    outs = [torch.empty_like(x.q) for x in bs]
    launches = [lambda x=x, o=o: paged.paged_attention(plan, x.q, x.k_cache, x.v_cache, x.block_table, out=o)
                for x, o in zip(bs, outs)]
    per, wall = _events_time(launches, warmup, steps)
    step = _graph_time(launches, warmup, steps)
    nbytes = workloads.decode_bytes(b)
    res = {
        "bytes_per_launch": nbytes, "flops_per_launch": workloads.attention_flops(b),
        # graph replay: launches run back to back, so the step time is the
        # launch's duration on the stream (decode kernel + split merge if any)
        "ms_per_step": step, "kernel_ms_mean": step,
        "gbs": nbytes / (step * 1e-3) / 1e9, "kernel_gbs": nbytes / (step * 1e-3) / 1e9,
        # eager launches from Python, for comparison (host launch cost included)
        "eager_ms_per_step": wall, "eager_launch_ms_mean": statistics.mean(per),
        "eager_launch_ms_median": statistics.median(per),
        "split_tokens": plan.info["split_tokens"], "work_items": plan.info["work_items"],
        "heads_per_wg": plan.info["heads_per_wg"], "decode_waves": plan.info["decode_waves"],
        "pool_copies": copies,
    }
    res["hbm_frac"] = res["kernel_gbs"] / HBM_PEAK_GBS
    return res, bs[0], plan


def bench_prefill(b, copies, warmup, steps, dev):
    bs = _copies(b, copies, dev, on_device=True)
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=b.num_q_heads, num_kv_heads=b.num_kv_heads,
                               head_dim=b.head_dim, block_size=b.block_size, dtype=b.dtype, device=dev)
    outs = [torch.empty_like(x.q) for x in bs]
    pos = [torch.cat([torch.arange(c, c + q) for c, q in zip(b.ctx_lens, b.q_lens)]).to(dev) for _ in bs]

    def write(x, p):
        paged.rope_kv_write(x.k_new, x.v_new, x.cos, x.sin, x.k_cache, x.v_cache, x.slot_mapping, rope_rows=p)

    def attn(x, o):
        paged.paged_attention(plan, x.q, x.k_cache, x.v_cache, x.block_table, out=o, rope=(x.cos, x.sin, "position"))

    wper, _ = _events_time([lambda x=x, p=p: write(x, p) for x, p in zip(bs, pos)], warmup, steps)
    aper, _ = _events_time([lambda x=x, o=o: attn(x, o) for x, o in zip(bs, outs)], warmup, steps)
    _, wall = _events_time([lambda x=x, p=p, o=o: (write(x, p), attn(x, o)) for x, p, o in zip(bs, pos, outs)],
                           warmup, steps)
    flops = workloads.attention_flops(b)
    am = statistics.mean(aper)
    wm = statistics.mean(wper)
    wb = workloads.rope_write_bytes(b)
    return {
        "flops_per_launch": flops, "attn_kernel_ms_mean": am, "tflops": flops / (am * 1e-3) / 1e12,
        "mfma_frac": flops / (am * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
        "rope_write_ms_mean": wm, "rope_write_gbs": wb / (wm * 1e-3) / 1e9,
        "step_ms": wall, "step_tflops": flops / (wall * 1e-3) / 1e12,
        "tokens": b.rows, "work_items": plan.info["work_items"],
    }


def bench_qkv(n_tokens, hidden, Hq, Hkv, D, weight_copies, warmup, steps, dev, seed=5):
    """Fused QKV projection + RoPE + KV write (``gllm_qkv_rope_kv_write``) vs
    the unfused path (three bf16 GEMMs through torch/hipBLASLt + the RoPE/KV
    write kernel), both graph-timed.  Weight copies are rotated so a decode
    step's weights come from HBM, not the 256 MB Infinity Cache."""
    g = torch.Generator(device=dev).manual_seed(seed)
    bf = torch.bfloat16
    x = torch.randn(n_tokens, hidden, device=dev, generator=g, dtype=torch.float32).to(bf)
    ws = []
    for _ in range(weight_copies):
        w = [(torch.randn(h * D, hidden, device=dev, generator=g) / hidden ** 0.5).to(bf) for h in (Hq, Hkv, Hkv)]
        ws.append((w, [t.t().contiguous() for t in w]))        # [out, in] and its transpose for torch.mm
    max_pos = 8192
    inv = 500000.0 ** (-2 * torch.arange(D // 2, device=dev) / D)
    ang = torch.arange(max_pos, device=dev).unsqueeze(1) * inv
    cos, sin = torch.cos(ang).to(bf), torch.sin(ang).to(bf)
    pos = torch.randint(0, max_pos, (n_tokens,), device=dev, generator=g)
    ns = n_tokens + 16
    slots = torch.randperm(ns, device=dev, generator=g)[:n_tokens].contiguous()
    kc = torch.zeros(ns, Hkv, D, dtype=bf, device=dev)
    vc = torch.zeros_like(kc)
    q_out = torch.empty(n_tokens, Hq, D, dtype=bf, device=dev)

    def fused(w):
        paged.qkv_rope_kv_write(x, w[0], w[1], w[2], cos, sin, kc, vc, slots, q_out=q_out, rope_rows=pos)

    def unfused(wt):
        q = torch.mm(x, wt[0])
        k = torch.mm(x, wt[1])
        v = torch.mm(x, wt[2])
        paged.rope_kv_write(k.view(n_tokens, Hkv, D), v.view(n_tokens, Hkv, D), cos, sin, kc, vc, slots,
                            q=q.view(n_tokens, Hq, D), q_out=q_out, rope_rows=pos)

    tf = _graph_time([lambda w=w: fused(w) for w, _ in ws], warmup, steps)
    tu = _graph_time([lambda wt=wt: unfused(wt) for _, wt in ws], warmup, steps)
    flops = 2 * n_tokens * (Hq + 2 * Hkv) * D * hidden
    wbytes = (Hq + 2 * Hkv) * D * hidden * 2
    iobytes = wbytes + n_tokens * hidden * 2 + n_tokens * (Hq + 2 * Hkv) * D * 2
    return {"tokens": n_tokens, "hidden": hidden, "fused_ms": tf, "unfused_ms": tu, "speedup": tu / tf,
            "tflops": flops / (tf * 1e-3) / 1e12, "mfma_frac": flops / (tf * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
            "gbs": iobytes / (tf * 1e-3) / 1e9, "hbm_frac": iobytes / (tf * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "weight_copies": weight_copies}


def bench_metadata(b: workloads.PagedBatch, warmup, steps, dev, cpu: bool):
    """Device metadata builder (query-row slots + positions + cu_seqlens) on
    one batch; with ``cpu`` also the reference path's host builder
    (llm.py:245-293: per-row loop, left-padded slot mapping, dense 0/-inf
    bias), restated by the oracle, on the same lengths and table."""
    bt = b.block_table if b.block_table.is_cuda else b.block_table.to(dev)
    sl = torch.tensor(b.seq_lens, dtype=torch.int32, device=dev)
    ql = torch.tensor(b.q_lens, dtype=torch.int32, device=dev)
    launches = [lambda: paged.build_metadata(bt, sl, ql, b.block_size, num_rows=b.rows)]
    step = _graph_time(launches, warmup, steps)
    res = {"rows": b.rows, "seqs": len(b.q_lens), "gpu_us": step * 1e3}
    if cpu:
        from oracle import metadata as om
        import time
        bt_np = bt.cpu().numpy()
        ts = []
        for i in range(4):
            t0 = time.perf_counter()
            om.build_metadata(b.ctx_lens, b.q_lens, bt_np, b.block_size, dtype=b.dtype)
            ts.append(time.perf_counter() - t0)
        res["cpu_reference_ms"] = statistics.median(ts[1:]) * 1e3
    return res


def cpu_baseline_decode(x: workloads.PagedBatch, nbytes: int):
    """The reference's CPU path for config (b): padded slot mapping + 0/-inf
    bias (llm.py:245-274), dense gather with the dtype cast (attention.py:
    165-170), GQA expand + softmax attention (reference_attention.py), fp32."""
    from oracle import attention as oa
    from oracle import metadata as om
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    bt = x.block_table.cpu().numpy()
    meta = om.build_metadata(x.ctx_lens, x.q_lens, bt, x.block_size, torch.float32)
    kc = x.k_cache.cpu()
    vc = x.v_cache.cpu()
    q = x.q.cpu().view(len(x.q_lens), 1, x.num_q_heads, x.head_dim).float()

    def run():
        k = oa.kv_gather(kc, meta.slot_mapping, torch.float32)
        v = oa.kv_gather(vc, meta.slot_mapping, torch.float32)
        return oa.reference_attention(q, k, v, meta.bias)

    run()
    ts = []
    for _ in range(3):
        t = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t)
    med = statistics.median(ts)
    return {"value": nbytes / med / 1e9, "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"full config (b) batch, median of 3 after 1 warm-up, {med * 1e3:.1f} ms/batch, "
                      f"fp32 torch on {platform.processor() or platform.machine()}"}


def _traffic(name: str):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, scaled by a copy-kernel calibration), if a committed summary
    holds it."""
    p = os.path.join(ROOT, "profiles", f"traffic_{name}.txt")
    if not os.path.exists(p):
        return None
    for line in open(p):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--configs", default="b,c,d,e")
    ap.add_argument("--split", type=int, default=0, help="decode split tokens (0 = planner's choice)")
    ap.add_argument("--hw", type=int, default=0, help="kv heads per decode workgroup (0 = planner's choice)")
    ap.add_argument("--copies", type=int, default=4, help="KV pool copies rotated for config (b)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate", action="store_true",
                    help="also run a plain 256 MiB device copy (known bytes) for counter calibration")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: --gpus must be 1 "
                                   "(multi-GPU sharding is described in DESIGN.md, not built)"}))
        sys.exit(2)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    cfgs = args.configs.split(",")
    extra = {}
    head = None
    if "b" in cfgs:
        b = workloads.config_b()
        head, x0, _ = bench_decode(b, args.copies, args.warmup, args.steps, args.split, dev, args.hw)
        extra["decode_1b"] = head
        extra["metadata_decode_1b"] = bench_metadata(x0, args.warmup, args.steps, dev, not args.no_cpu)
        # the same batch over an fp8 (e4m3fn) KV pool: half the K/V bytes
        b8 = workloads.config_b()
        b8.kv_dtype = torch.float8_e4m3fn
        r8, _, _ = bench_decode(b8, args.copies, args.warmup, args.steps, args.split, dev, args.hw)
        r8["speedup_vs_bf16_kv"] = head["ms_per_step"] / r8["ms_per_step"]
        extra["decode_1b_fp8kv"] = r8
        torch.cuda.empty_cache()
        # fused QKV projection + RoPE + KV write for the same 64 decode tokens (1B layer)
        extra["qkv_decode_1b"] = bench_qkv(64, 2048, 32, 8, 64, 24, args.warmup, args.steps, dev)
        torch.cuda.empty_cache()
    if "c" in cfgs:
        extra["prefill_8b"] = bench_prefill(workloads.config_c(), 2, args.warmup, args.steps, dev)
        torch.cuda.empty_cache()
        # fused QKV projection + RoPE + KV write for config (c)'s tokens (8B layer)
        extra["qkv_prefill_8b"] = bench_qkv(workloads.config_c().rows, 4096, 32, 8, 128, 2, args.warmup,
                                            max(5, args.steps // 3), dev)
        torch.cuda.empty_cache()
    if "d" in cfgs:
        r, xd, _ = bench_decode(workloads.config_d(), 1, args.warmup, args.steps, args.split, dev, args.hw)
        extra["mixed_8b"] = r
        extra["metadata_mixed_8b"] = bench_metadata(xd, args.warmup, args.steps, dev, False)
        del xd
        torch.cuda.empty_cache()
        # the decode sequences of the same batch alone: decode at the 8B head shape
        d = workloads.config_d()
        dd = workloads.PagedBatch("decode_8b", d.ctx_lens[:256], d.q_lens[:256], d.num_q_heads, d.num_kv_heads,
                                  d.head_dim, d.block_size, d.num_blocks, d.dtype, rope_theta=d.rope_theta)
        r, _, _ = bench_decode(dd, 1, args.warmup, args.steps, args.split, dev, args.hw)
        extra["decode_8b"] = r
        torch.cuda.empty_cache()
    if "e" in cfgs:
        r, _, _ = bench_decode(workloads.config_e(), 1, args.warmup, max(5, args.steps // 3), args.split, dev, args.hw)
        extra["long_decode_70b"] = r
        torch.cuda.empty_cache()
    if args.calibrate:
        src = torch.empty(128 << 20, dtype=torch.bfloat16, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
    cpu = None
    if head is not None and not args.no_cpu:
        cpu = cpu_baseline_decode(x0, head["bytes_per_launch"])
    line = {
        "metric": "decode attn GB/s (% HBM peak); prefill attn TFLOP/s (% MFMA peak), 8B GQA",
        "value": round(head["gbs"], 2) if head else None,
        "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 5) if head else None,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (seeded N(0,1) Q/K/V, random block tables)",
        "config": {"workload": "decode paged attention, Llama-3.2-1B heads: B 64, Hq 32 / Hkv 8, D 64, "
                               "bs 16, seq len U{128..2048}, 16384-block pool, 1 query token per sequence",
                   "global_batch": 64, "parallelism": "none (1 GPU)",
                   "launch": "the K timed steps captured in one HIP graph, 4 KV pool copies rotated"},
        "roofline": None if head is None else {
            "bound": "hbm", "achieved": round(head["kernel_gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(head["hbm_frac"], 4), "traffic": _traffic("decode_1b")},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
