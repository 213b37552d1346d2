"""Benchmark of the gLLM attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs d,c,b,a,e]

Prints ONE JSON line.  The headline (``value``) is benchmark config (d), the
metric's 8B GQA shape: one paged-attention launch over a mixed continuous
batch (256 decode sequences + 4 chunked prefills of 512 tokens, Llama-3.1-8B
heads), in GB/s of compulsory HBM bytes per launch, inputs resident in HBM.
A "step" is that launch (one layer's attention over the batch).  Timing: a
few steps are captured in one HIP graph (so graph-launch gaps do not count
as kernel time) and the graph is replayed K times (K >= 50 by default), each
replay bracketed by HIP events on the stream the kernels run on; the
reported step time is the median over the replays of replay time / steps.  Configs (c) prefill
(TFLOP/s against the bf16 MFMA peak), (d)'s decodes alone, (e) long decode
and (b) 1B decode are reported in ``extra``, each with its own roofline and
CPU-baseline objects.  The CPU baseline times the reference's path (dense KV
gather through the slot mapping, GQA expand, softmax attention with the
0/-inf bias; fp32 torch on every host core) per sequence (B = 1, no padding)
and sums, on the same inputs copied from the GPU.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from gllm_amd import _lib, paged, workloads  # noqa: E402

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


# ------------------------------------------------------------------ timing
def graph_reps(launches, warmup: int, reps: int, inner: int):
    """``inner`` steps (``launches[i % n]``, so KV-pool copies rotate inside
    the graph) captured in one HIP graph, replayed ``warmup`` times untimed,
    then ``reps`` times, each replay bracketed by HIP events on the current
    stream (the one the kernels are launched on).  Returns the per-step ms of
    every replay and the mean per-step ms over the whole timed region
    (synchronised on both sides)."""
    cur = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    side.wait_stream(cur)
    with torch.cuda.stream(side):              # first launches outside capture
        for f in launches:
            f()
    cur.wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(inner):
            launches[i % len(launches)]()
    for _ in range(max(1, warmup)):
        g.replay()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record()
    for s, e in ev:
        s.record()
        g.replay()
        e.record()
    t1.record()
    torch.cuda.synchronize()
    per = [s.elapsed_time(e) / inner for s, e in ev]
    return per, t0.elapsed_time(t1) / (reps * inner)


def eager_reps(launches, warmup: int, reps: int):
    """Eager launches from Python (host launch cost included), per-launch
    HIP events; returns the per-launch ms."""
    for i in range(warmup):
        launches[i % len(launches)]()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for i, (s, e) in enumerate(ev):
        s.record()
        launches[i % len(launches)]()
        e.record()
    torch.cuda.synchronize()
    return [s.elapsed_time(e) for s, e in ev]


def _stats(per, wall):
    return {"ms_per_step": statistics.median(per), "ms_mean": statistics.mean(per), "ms_min": min(per),
            "ms_max": max(per), "reps": len(per), "ms_per_step_region_mean": wall}


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


def roofline_hbm(nbytes: int, ms: float, traffic_name: str):
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": _traffic(traffic_name)}


def roofline_mfma(flops: int, ms: float, traffic_name: str):
    tf = flops / (ms * 1e-3) / 1e12
    return {"bound": "mfma", "achieved": round(tf, 2), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tf / BF16_PEAK_TFLOPS, 4), "traffic": _traffic(traffic_name)}


# ------------------------------------------------------------------ GPU legs
def _copies(b: workloads.PagedBatch, n: int, dev):
    """n independent pools (same lengths, own values and tables) so repeated
    launches stream HBM rather than the 256 MB Infinity Cache."""
    out = []
    for i in range(n):
        c = workloads.PagedBatch(**{k: getattr(b, k) for k in (
            "name", "ctx_lens", "q_lens", "num_q_heads", "num_kv_heads", "head_dim", "block_size",
            "num_blocks", "dtype", "rope_theta", "kv_dtype")})
        out.append(workloads.materialize(c, dev, values_on_device=True, seed=2 + i))
    return out


def bench_paged(b, copies, warmup, reps, inner, dev, split=0, hw=0, eager=True, rope=False):
    """One paged-attention launch per step over batch ``b`` (decode, mixed or
    prefill); with ``rope`` q is rotated on load (RoPE table rows c_i + r)."""
    xs = _copies(b, copies, dev)
    t = time.perf_counter()
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=b.num_q_heads, num_kv_heads=b.num_kv_heads,
                               head_dim=b.head_dim, block_size=b.block_size, dtype=b.dtype, device=dev,
                               split_tokens=split, heads_per_wg=hw)
    torch.cuda.synchronize()
    plan_ms = (time.perf_counter() - t) * 1e3
    outs = [torch.empty_like(x.q) for x in xs]
    launches = [lambda x=x, o=o: paged.paged_attention(plan, x.q, x.k_cache, x.v_cache, x.block_table, out=o,
                                                       rope=(x.cos, x.sin, "position") if rope else None)
                for x, o in zip(xs, outs)]
    per, wall = graph_reps(launches, warmup, reps, inner)
    res = _stats(per, wall)
    res.update({"bytes_per_launch": workloads.decode_bytes(b), "flops_per_launch": workloads.attention_flops(b),
                "graph_steps_per_replay": inner, "pool_copies": copies, "plan_create_upload_ms": plan_ms,
                **{k: plan.info[k] for k in ("work_items", "split_tokens", "heads_per_wg", "decode_segments")}})
    if eager:
        ep = eager_reps(launches, warmup, reps)
        res["eager_ms_median"] = statistics.median(ep)
    return res, xs[0], outs[0]


def bench_prefill_step(b, x, warmup, reps, dev):
    """Config (c) as one step: the RoPE + KV write of the batch's new tokens
    (K rotated and written into its pages) followed by the paged attention
    launch with q rotated on load, both in one graph step.  Work: the
    attention flops (MFMA roofline) and the step's compulsory bytes (the
    write's bytes plus the attention's)."""
    pos = torch.cat([torch.arange(c, c + q) for c, q in zip(b.ctx_lens, b.q_lens)]).to(dev)
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=b.num_q_heads, num_kv_heads=b.num_kv_heads,
                               head_dim=b.head_dim, block_size=b.block_size, dtype=b.dtype, device=dev)
    out = torch.empty_like(x.q)

    def step():
        paged.rope_kv_write(x.k_new, x.v_new, x.cos, x.sin, x.k_cache, x.v_cache, x.slot_mapping, rope_rows=pos)
        paged.paged_attention(plan, x.q, x.k_cache, x.v_cache, x.block_table, out=out,
                              rope=(x.cos, x.sin, "position"))
    per, wall = graph_reps([step], warmup, reps, 4)
    ms = statistics.median(per)
    flops = workloads.attention_flops(b)
    nbytes = workloads.rope_write_bytes(b) + workloads.decode_bytes(b)
    r = roofline_mfma(flops, ms, "prefill_step_8b")
    return {"ms_per_step": ms, "launches_per_step": 2, "flops_per_step": flops, "bytes_per_step": nbytes,
            "hbm_gbs": nbytes / (ms * 1e-3) / 1e9, "roofline": r}


def bench_rope_write(b, x, warmup, reps, dev):
    """The fused RoPE + KV write of the batch's new tokens (graph-timed)."""
    pos = torch.cat([torch.arange(c, c + q) for c, q in zip(b.ctx_lens, b.q_lens)]).to(dev)
    f = [lambda: paged.rope_kv_write(x.k_new, x.v_new, x.cos, x.sin, x.k_cache, x.v_cache, x.slot_mapping,
                                     rope_rows=pos)]
    per, wall = graph_reps(f, warmup, reps, 4)
    nb = workloads.rope_write_bytes(b)
    ms = statistics.median(per)
    return {"ms_per_step": ms, "bytes": nb, "gbs": nb / (ms * 1e-3) / 1e9, "hbm_frac": nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}


def bench_qkv(n_tokens, hidden, Hq, Hkv, D, weight_copies, warmup, reps, dev, seed=5):
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

    def fused(w):       # the fused kernel itself
        paged.qkv_rope_kv_write(x, w[0], w[1], w[2], cos, sin, kc, vc, slots, q_out=q_out, rope_rows=pos,
                                unfused_from=None)

    def dispatched(w):  # the library entry as callers use it (size-based choice of path)
        paged.qkv_rope_kv_write(x, w[0], w[1], w[2], cos, sin, kc, vc, slots, q_out=q_out, rope_rows=pos)

    def unfused(wt):
        q = torch.mm(x, wt[0])
        k = torch.mm(x, wt[1])
        v = torch.mm(x, wt[2])
        paged.rope_kv_write(k.view(n_tokens, Hkv, D), v.view(n_tokens, Hkv, D), cos, sin, kc, vc, slots,
                            q=q.view(n_tokens, Hq, D), q_out=q_out, rope_rows=pos)

    inner = weight_copies
    tf = statistics.median(graph_reps([lambda w=w: fused(w) for w, _ in ws], warmup, reps, inner)[0])
    td = statistics.median(graph_reps([lambda w=w: dispatched(w) for w, _ in ws], warmup, reps, inner)[0])
    tu = statistics.median(graph_reps([lambda wt=wt: unfused(wt) for _, wt in ws], warmup, reps, inner)[0])
    flops = 2 * n_tokens * (Hq + 2 * Hkv) * D * hidden
    wbytes = (Hq + 2 * Hkv) * D * hidden * 2
    iobytes = wbytes + n_tokens * hidden * 2 + n_tokens * (Hq + 2 * Hkv) * D * 2
    return {"tokens": n_tokens, "hidden": hidden, "fused_ms": tf, "dispatched_ms": td, "unfused_ms": tu,
            "path": "unfused" if n_tokens >= paged.QKV_UNFUSED_FROM else "fused",
            "speedup": tu / td, "fused_kernel_speedup": tu / tf,
            "tflops": flops / (tf * 1e-3) / 1e12, "mfma_frac": flops / (tf * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
            "gbs": iobytes / (tf * 1e-3) / 1e9, "hbm_frac": iobytes / (tf * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "weight_copies": weight_copies}


def bench_metadata(b: workloads.PagedBatch, warmup, reps, dev, cpu: bool):
    """Device metadata builder (query-row slots + positions + cu_seqlens) on
    one batch; with ``cpu`` also the reference path's host builder
    (llm.py:245-293: per-row loop, left-padded slot mapping, dense 0/-inf
    bias), restated by the oracle, on the same lengths and table."""
    bt = b.block_table if b.block_table.is_cuda else b.block_table.to(dev)
    sl = torch.tensor(b.seq_lens, dtype=torch.int32, device=dev)
    ql = torch.tensor(b.q_lens, dtype=torch.int32, device=dev)
    launches = [lambda: paged.build_metadata(bt, sl, ql, b.block_size, num_rows=b.rows)]
    per, _ = graph_reps(launches, warmup, reps, 16)
    res = {"rows": b.rows, "seqs": len(b.q_lens), "gpu_us": statistics.median(per) * 1e3}
    if cpu:
        from oracle import metadata as om
        bt_np = bt.cpu().numpy()
        ts = []
        for _ in range(4):
            t0 = time.perf_counter()
            om.build_metadata(b.ctx_lens, b.q_lens, bt_np, b.block_size, dtype=b.dtype)
            ts.append(time.perf_counter() - t0)
        res["cpu_reference_ms"] = statistics.median(ts[1:]) * 1e3
    return res


def bench_decode_step(dtype, warmup, reps, dev):
    """One decode step of a config (a)-shaped model's attention path (16
    layers of Llama-3.2-1B heads, 8 sequences, block size 16): per layer the
    RoPE + KV write and the paged attention (``Attention.attention``: one
    launch per layer that also writes the new K/V, or two where the fused
    write does not apply).  Eager launches from Python vs the same step
    captured in one HIP graph; returns both per-step times (median over
    ``reps``)."""
    import gllm_amd
    L, Hq, Hkv, D, bs, B = 16, 32, 8, 64, 16, 8
    g = torch.Generator().manual_seed(31)
    ctx = torch.randint(20, 200, (B,), generator=g).tolist()
    seq = [c + 1 for c in ctx]
    cache = gllm_amd.PagedKVCache(L, Hkv, D, bs, B, 256, dtype, dev)
    cache.physical_kv_cache.normal_()
    bt = workloads.block_tables(seq, bs, cache.num_blocks).to(dev)
    rows = torch.arange(B)
    pos = torch.tensor(ctx)
    qsm = (bt.cpu()[rows, pos // bs].to(torch.int64) * bs + pos % bs).view(B, 1).to(dev)
    gm = gllm_amd.AttentionMetadata(query_lens=torch.ones(B, dtype=torch.int32, device=dev),
                                    seq_lens=torch.tensor(seq, dtype=torch.int32, device=dev), max_seq_len=max(seq),
                                    block_table=bt, slot_mapping=None, query_slot_mapping=qsm, bias=None,
                                    block_size=bs)
    ang = pos.unsqueeze(1) * 500000.0 ** (-2 * torch.arange(D // 2) / D)
    cos, sin = torch.cos(ang).to(dtype).view(B, 1, -1).to(dev), torch.sin(ang).to(dtype).view(B, 1, -1).to(dev)

    class Cfg:
        num_attn_heads, num_kv_heads, head_dim, hidden_size = Hq, Hkv, D, Hq * D

    Cfg.dtype = dtype
    atts = [gllm_amd.Attention(li, Cfg, {f"model.layers.{li}.self_attn.{n}_proj.weight": torch.zeros(1)
                                         for n in "qkvo"}) for li in range(L)]
    qs = [torch.randn(B, 1, Hq, D, device=dev).to(dtype) for _ in range(L)]
    ks = [torch.randn(B, 1, Hkv, D, device=dev).to(dtype) for _ in range(L)]
    vs = [torch.randn(B, 1, Hkv, D, device=dev).to(dtype) for _ in range(L)]

    def step():
        for li in range(L):
            atts[li].attention(qs[li], ks[li], vs[li], cos, sin, cache.get_layer_kv_cache(li), gm)

    step()                                         # builds the plan once
    torch.cuda.synchronize()
    from gllm_amd import paged
    fused = paged.fused_kv_write_ok(gm._gllm_plan, cache.physical_kv_cache.dtype)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for s_, e_ in ev:
        s_.record()
        step()
        e_.record()
    torch.cuda.synchronize()
    eager = statistics.median(s_.elapsed_time(e_) for s_, e_ in ev)
    per, _ = graph_reps([step], warmup, reps, 1)
    graph = statistics.median(per)
    return {"layers": L, "seqs": B, "dtype": str(dtype).replace("torch.", ""), "launches_per_step": L if fused else 2 * L,
            "kv_write_fused": fused,
            "eager_ms_per_step": eager, "graph_ms_per_step": graph, "saving_ms": eager - graph,
            "speedup": eager / graph}


def progress(what: str) -> None:
    """One line per stage on stderr (the JSON result line stays alone on stdout)."""
    print(f"[bench] {what}", file=sys.stderr, flush=True)


def bench_box_ceilings(dev, warmup, reps):
    """What this box reaches on plain patterns, as context for the roofline
    fractions (not the peaks they are priced against): a device copy of 2 GiB
    (torch's copy kernel; bytes read + written), the time per graph node of a one-element kernel (the launch floor of a
    graph-replayed step) and a bf16 8192^3 GEMM (torch.mm -> hipBLASLt)."""
    src = torch.empty(1 << 30, dtype=torch.bfloat16, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    per, _ = graph_reps([lambda: dst.copy_(src)], warmup, reps, 1)
    copy_ms = statistics.median(per)
    del src, dst
    cb = 2 * (2 << 30)
    out = {"copy_2gib_gbs": cb / (copy_ms * 1e-3) / 1e9,
           "copy_frac_of_hbm_peak": cb / (copy_ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
    # launch floor: a one-element kernel per graph node, 32 nodes per graph
    one = torch.zeros(1, device=dev)
    per, _ = graph_reps([lambda: one.add_(1.0)], warmup, max(5, reps // 2), 32)
    out["tiny_kernel_graph_us"] = statistics.median(per) * 1e3
    del one
    a = torch.randn(8192, 8192, device=dev).to(torch.bfloat16)
    bm = torch.randn(8192, 8192, device=dev).to(torch.bfloat16)
    per, _ = graph_reps([lambda: torch.mm(a, bm)], warmup, max(5, reps // 4), 1)
    gemm_ms = statistics.median(per)
    del a, bm
    torch.cuda.empty_cache()
    out["gemm_bf16_8192_tflops"] = 2 * 8192 ** 3 / (gemm_ms * 1e-3) / 1e12
    out["gemm_frac_of_mfma_peak"] = out["gemm_bf16_8192_tflops"] / BF16_PEAK_TFLOPS
    return out


def bench_plan_host(b: workloads.PagedBatch, reps: int, dev):
    """Host cost of one engine step's plan (what plan_for pays once per step):
    create (planner + pinned staging from the library's pool), device
    workspace (torch's caching allocator), upload (an enqueued copy), destroy
    (staging back to the pool).  Median over ``reps`` after a warm-up."""
    def once():
        t = time.perf_counter()
        p = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=b.num_q_heads, num_kv_heads=b.num_kv_heads,
                                head_dim=b.head_dim, block_size=b.block_size, dtype=b.dtype, device=dev)
        del p
        return (time.perf_counter() - t) * 1e3
    for _ in range(3):
        once()
    torch.cuda.synchronize()
    ts = [once() for _ in range(reps)]
    torch.cuda.synchronize()
    return {"seqs": len(b.q_lens), "host_ms_median": statistics.median(ts), "host_ms_max": max(ts)}


# ------------------------------------------------------------------ CPU baseline
def _cpu_setup():
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    return cores


def cpu_baseline_per_sequence(x: workloads.PagedBatch, seqs: list[int], unit: str, what: str):
    """The reference's CPU path, one sequence at a time (B = 1: no padding),
    on the batch's own inputs copied from the GPU: per-sequence metadata
    (llm.py:245-274), dense K/V gather through the slot mapping with the
    dtype cast (attention.py:165-170), q rotated (attention.py:76-119) when the
    batch carries a RoPE table, then GQA expand + softmax attention with the
    0/-inf bias (reference_attention.py:5-51), fp32 torch on every host core.
    The metadata build is outside the timed region (once per engine step);
    one untimed warm-up pass over ``seqs``, then the median of 3 timed
    passes.  Work per sequence uses the same formulas as the GPU figure, so
    ``value`` is directly comparable."""
    from oracle import attention as oa
    from oracle import metadata as om
    from oracle import rope as orope
    cores = _cpu_setup()
    bs, Hkv, D = x.block_size, x.num_kv_heads, x.head_dim
    rope = x.cos is not None
    cos_c = x.cos.cpu().float() if rope else None
    sin_c = x.sin.cpu().float() if rope else None
    bt_all = x.block_table.cpu()
    kv_view = lambda t: t.view(-1, bs, Hkv, D)
    jobs = []
    for i in seqs:
        c, q, r0 = x.ctx_lens[i], x.q_lens[i], x.q_row_start[i]
        L = c + q
        nb = -(-L // bs)
        blocks = bt_all[i, :nb].to(torch.int64)
        kc = kv_view(x.k_cache)[blocks.to(x.k_cache.device)].cpu().reshape(-1, Hkv, D)   # the sequence's pages
        vc = kv_view(x.v_cache)[blocks.to(x.v_cache.device)].cpu().reshape(-1, Hkv, D)
        meta = om.build_metadata([c], [q], torch.arange(nb, dtype=torch.int32).numpy()[None], bs, torch.float32)
        qq = x.q[r0:r0 + q].cpu().float().unsqueeze(0)
        pos = torch.arange(c, c + q)
        jobs.append((kc, vc, meta, qq, pos))

    def run(job):
        kc, vc, meta, qq, pos = job
        if rope:
            qq = orope.apply_rope(qq, cos_c[pos].unsqueeze(0), sin_c[pos].unsqueeze(0))
        k = oa.kv_gather(kc, meta.slot_mapping, torch.float32)
        v = oa.kv_gather(vc, meta.slot_mapping, torch.float32)
        return oa.reference_attention(qq, k, v, meta.bias)

    passes = []
    for rep in range(4):                       # pass 0 is the warm-up
        t = time.perf_counter()
        for job in jobs:
            run(job)
        if rep:
            passes.append(time.perf_counter() - t)
    sec = statistics.median(passes)
    sub = workloads.PagedBatch("sample", [x.ctx_lens[i] for i in seqs], [x.q_lens[i] for i in seqs],
                               x.num_q_heads, Hkv, D, bs, x.num_blocks, x.dtype, kv_dtype=x.kv_dtype)
    work = workloads.decode_bytes(sub) / 1e9 if unit == "GB/s" else workloads.attention_flops(sub) / 1e12
    return {"value": work / sec, "unit": unit, "cores": cores, "kind": "port",
            "sample": f"{what}: {len(seqs)} of {len(x.q_lens)} sequences, one at a time (B=1), "
                      f"median of 3 timed passes after 1 warm-up pass ({', '.join(f'{v:.2f}' for v in passes)} s) "
                      f"for {work:.4g} {'GB' if unit == 'GB/s' else 'TFLOP'} of the same "
                      f"formula as the GPU figure; fp32 torch on {cores} threads of {cpu_model()}"}


def cpu_baseline_batched(x: workloads.PagedBatch):
    """Config (b): the reference's CPU path on the whole batch at once, as
    the engine runs it (padded slot mapping + 0/-inf bias, llm.py:245-274;
    dense gather, attention.py:165-170; GQA expand + softmax attention,
    reference_attention.py), fp32; median of 3 after 1 warm-up."""
    from oracle import attention as oa
    from oracle import metadata as om
    cores = _cpu_setup()
    bt = x.block_table.cpu().numpy()
    meta = om.build_metadata(x.ctx_lens, x.q_lens, bt, x.block_size, torch.float32)
    kc, vc = x.k_cache.cpu(), x.v_cache.cpu()
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
    return {"value": workloads.decode_bytes(x) / med / 1e9, "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"full config (b) batch (B=64, padded, as the engine batches it), median of 3 after "
                      f"1 warm-up, {med * 1e3:.1f} ms/batch; fp32 torch on {cores} threads of {cpu_model()}"}


# ------------------------------------------------------------------ main
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=60, help="timed steps (graph replays) of the headline config")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--configs", default="d,c,b,a,e")
    ap.add_argument("--split", type=int, default=0, help="decode split tokens (0 = planner's choice)")
    ap.add_argument("--hw", type=int, default=0, help="kv heads per decode workgroup (0 = planner's choice)")
    ap.add_argument("--copies", type=int, default=4, help="KV pool copies rotated for config (b)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-ceilings", action="store_true", help="skip the copy / GEMM reference measurements")
    ap.add_argument("--calibrate", action="store_true",
                    help="also run a plain 256 MiB device copy (known bytes) for counter calibration")
    ap.add_argument("--qkv-sweep", action="store_true",
                    help="only time the QKV projection path over token counts at the 1B / 8B / 70B layer shapes "
                         "(one JSON line) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: --gpus must be 1 (nothing multi-GPU is "
                                   "built; the path would shard by sequence or kv head with no exchange)"}))
        sys.exit(2)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.qkv_sweep:
        rows = []
        for name, hid, hq, hkv, hd in (("1B", 2048, 32, 8, 64), ("8B", 4096, 32, 8, 128), ("70B", 8192, 64, 8, 128)):
            for n in (1, 16, 32, 64, 128, 256, 512, 1024, 2048):
                r = bench_qkv(n, hid, hq, hkv, hd, 24 if n <= 256 else 4, args.warmup, 15, dev)
                rows.append({"layer": name, **{k: r[k] for k in ("tokens", "fused_ms", "dispatched_ms", "unfused_ms",
                                                                 "hbm_frac", "mfma_frac")}})
                progress(f"qkv {name} n={n}: fused {r['fused_ms'] * 1e3:.1f} us, dispatched "
                         f"{r['dispatched_ms'] * 1e3:.1f} us, unfused {r['unfused_ms'] * 1e3:.1f} us")
        print(json.dumps({"qkv_sweep": rows}))
        return
    cfgs = args.configs.split(",")
    reps = max(args.steps, 1)
    cpu = not args.no_cpu
    extra = {}
    head = None
    head_cpu = None
    if "d" in cfgs:
        progress("config (d)")
        d = workloads.config_d()
        head, xd, _ = bench_paged(d, 1, args.warmup, reps, 4, dev, args.split, args.hw)
        head["roofline"] = roofline_hbm(head["bytes_per_launch"], head["ms_per_step"], "mixed_8b")
        # the chunked-prefill part of (d): its flops over the mixed launch's
        # time, and the 4 chunks launched alone (prefill items only)
        dch = workloads.PagedBatch("mixed_8b_chunks", d.ctx_lens[256:], d.q_lens[256:], d.num_q_heads,
                                   d.num_kv_heads, d.head_dim, d.block_size, d.num_blocks, d.dtype,
                                   rope_theta=d.rope_theta)
        cf = workloads.attention_flops(dch)
        rc, _, _ = bench_paged(dch, 2, args.warmup, reps, 4, dev, eager=False)
        head["chunk_part"] = {
            "flops": cf, "share_of_launch_flops": cf / head["flops_per_launch"],
            "roofline_over_mixed_launch": roofline_mfma(cf, head["ms_per_step"], "none"),
            "alone": {"ms_per_step": rc["ms_per_step"], "work_items": rc["work_items"],
                      "roofline": roofline_mfma(cf, rc["ms_per_step"], "mixed_8b_chunks")}}
        extra["mixed_8b"] = head
        extra["metadata_mixed_8b"] = bench_metadata(xd, args.warmup, reps, dev, False)
        if cpu:
            head_cpu = cpu_baseline_per_sequence(xd, list(range(len(d.q_lens))), "GB/s", "all of config (d)")
        del xd
        torch.cuda.empty_cache()
        # the decode sequences of the same batch alone: decode at the 8B head shape
        dd = workloads.PagedBatch("decode_8b", d.ctx_lens[:256], d.q_lens[:256], d.num_q_heads, d.num_kv_heads,
                                  d.head_dim, d.block_size, d.num_blocks, d.dtype, rope_theta=d.rope_theta)
        r, _, _ = bench_paged(dd, 1, args.warmup, reps, 4, dev, args.split, args.hw, eager=False)
        r["roofline"] = roofline_hbm(r["bytes_per_launch"], r["ms_per_step"], "decode_8b")
        extra["decode_8b"] = r
        torch.cuda.empty_cache()
        # fused QKV projection + RoPE + KV write for (d)'s 256 decode tokens (8B layer)
        extra["qkv_decode_8b"] = bench_qkv(256, 4096, 32, 8, 128, 8, args.warmup, max(10, reps // 3), dev)
        torch.cuda.empty_cache()
    if "c" in cfgs:
        progress("config (c)")
        c = workloads.config_c()
        r, xc, _ = bench_paged(c, 2, args.warmup, reps, 4, dev, eager=False, rope=True)
        r["roofline"] = roofline_mfma(r["flops_per_launch"], r["ms_per_step"], "prefill_8b")
        r["rope_kv_write"] = bench_rope_write(c, xc, args.warmup, reps, dev)
        r["step"] = bench_prefill_step(c, xc, args.warmup, reps, dev)
        if cpu:
            r["cpu_baseline"] = cpu_baseline_per_sequence(xc, list(range(len(c.q_lens))), "TFLOP/s",
                                                          "all of config (c)")
        extra["prefill_8b"] = r
        del xc
        torch.cuda.empty_cache()
        # fused QKV projection + RoPE + KV write for config (c)'s tokens (8B layer)
        extra["qkv_prefill_8b"] = bench_qkv(c.rows, 4096, 32, 8, 128, 2, args.warmup, max(10, reps // 3), dev)
        torch.cuda.empty_cache()
    if "b" in cfgs:
        progress("config (b)")
        b = workloads.config_b()
        r, xb, _ = bench_paged(b, args.copies, args.warmup, reps, 2 * args.copies, dev, args.split, args.hw)
        r["roofline"] = roofline_hbm(r["bytes_per_launch"], r["ms_per_step"], "decode_1b")
        extra["metadata_decode_1b"] = bench_metadata(xb, args.warmup, reps, dev, cpu)
        if cpu:
            r["cpu_baseline"] = cpu_baseline_batched(xb)
        extra["decode_1b"] = r
        del xb
        # the same batch over an fp8 (e4m3fn) KV pool: half the K/V bytes
        b8 = workloads.config_b()
        b8.kv_dtype = torch.float8_e4m3fn
        r8, _, _ = bench_paged(b8, args.copies, args.warmup, reps, 2 * args.copies, dev, args.split, args.hw,
                               eager=False)
        r8["roofline"] = roofline_hbm(r8["bytes_per_launch"], r8["ms_per_step"], "decode_1b_fp8kv")
        r8["speedup_vs_bf16_kv"] = r["ms_per_step"] / r8["ms_per_step"]
        extra["decode_1b_fp8kv"] = r8
        torch.cuda.empty_cache()
        # fused QKV projection + RoPE + KV write for the same 64 decode tokens (1B layer)
        extra["qkv_decode_1b"] = bench_qkv(64, 2048, 32, 8, 64, 24, args.warmup, max(10, reps // 3), dev)
        # 16 decode tokens: the single-launch path (up to 32 tokens)
        extra["qkv_decode_1b_16"] = bench_qkv(16, 2048, 32, 8, 64, 24, args.warmup, max(10, reps // 3), dev)
        torch.cuda.empty_cache()
    if "a" in cfgs:
        progress("config (a)")
        # config (a)'s decode step: 16 layers x (RoPE + KV write, paged attention), eager vs one HIP graph
        extra["decode_step_1b_fp32"] = bench_decode_step(torch.float32, args.warmup, max(10, reps // 2), dev)
        extra["decode_step_1b_bf16"] = bench_decode_step(torch.bfloat16, args.warmup, max(10, reps // 2), dev)
        extra["plan_host_mixed_8b"] = bench_plan_host(workloads.config_d(), 50, dev)
        extra["plan_host_decode_1b"] = bench_plan_host(workloads.config_b(), 50, dev)
        torch.cuda.empty_cache()
    if "e" in cfgs:
        progress("config (e)")
        e = workloads.config_e()
        r, xe, _ = bench_paged(e, 1, args.warmup, max(10, reps // 2), 1, dev, args.split, args.hw, eager=False)
        r["roofline"] = roofline_hbm(r["bytes_per_launch"], r["ms_per_step"], "long_decode_70b")
        if cpu:
            r["cpu_baseline"] = cpu_baseline_per_sequence(xe, list(range(0, len(e.q_lens), 8)), "GB/s",
                                                          "every 8th sequence of config (e)")
        extra["long_decode_70b"] = r
        del xe
        torch.cuda.empty_cache()
    if not args.no_ceilings:
        progress("copy / GEMM reference")
        extra["box_ceilings"] = bench_box_ceilings(dev, args.warmup, max(10, reps // 3))
    if args.calibrate:
        src = torch.empty(128 << 20, dtype=torch.bfloat16, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
    line = {
        "metric": "decode attn GB/s (% HBM peak); prefill attn TFLOP/s (% MFMA peak), 8B GQA",
        "value": round(head["roofline"]["achieved"], 2) if head else None,
        "unit": "GB/s",
        "n_gpus": 1, "steps": reps, "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 5) if head else None,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (seeded N(0,1) Q/K/V, random block tables)",
        "config": {"workload": "config (d): mixed continuous batch, Llama-3.1-8B heads (Hq 32 / Hkv 8, D 128), "
                               "bs 16: 256 decode sequences with L log-uniform in [256, 8192] + 4 chunked "
                               "prefills of 512 tokens on contexts U{0..4096}, 131072-block pool, Q/K/V "
                               "N(0,1); one paged attention launch per step",
                   "global_batch": 260, "parallelism": "none (1 GPU)",
                   "timing": "4 steps captured in one HIP graph; per-step time = median over the timed "
                             "replays (HIP events on the launch stream around each replay) / 4"},
        "roofline": head["roofline"] if head else None,
        "cpu_baseline": head_cpu,
        "extra": extra,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
