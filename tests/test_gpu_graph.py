"""HIP graph capture of the attention launch, the way a serving loop runs a
decode step: capture once, replay every step.  The launch path only
enqueues kernels (no memset node, no allocation, no host wait), so it can be
captured.  Each replay must equal the eager result bit for bit (same
kernels, same inputs), with eager work and synchronisations between the
replays, and the eager result is itself checked against the CPU oracle."""
import pytest
import torch

from gllm_amd import paged
from tests.gpu_helpers import assert_close_bf16, make_batch, oracle_paged

pytestmark = pytest.mark.gpu

CASES = {
    # decode only, two heads per workgroup
    "decode": dict(ctx=[300, 17, 1500, 64, 900], ql=[1] * 5, Hq=32, Hkv=8, D=64, split=0),
    # decode with context splits (merge_splits_kernel runs in the graph too)
    "decode_split": dict(ctx=[4000, 33, 2500], ql=[1] * 3, Hq=64, Hkv=8, D=128, split=512),
    # page-balanced decode: split tickets drawn and re-armed inside the graph
    "decode_balanced": dict(ctx=[4000, 33, 2500, 700, 90], ql=[1] * 5, Hq=32, Hkv=8, D=64, split=paged.BALANCED),
    # mixed continuous batch: decodes plus two prefill chunks
    "mixed": dict(ctx=[700, 0, 250, 40], ql=[1, 90, 1, 33], Hq=32, Hkv=8, D=128, split=0),
    # mixed, page-balanced decode share: tickets re-armed inside the graph
    "mixed_balanced": dict(ctx=[4000, 0, 2500, 40, 900], ql=[1, 90, 1, 33, 1], Hq=32, Hkv=8, D=128,
                           split=paged.BALANCED),
}


@pytest.mark.parametrize("name", list(CASES))
def test_graph_replay_matches_eager(name):
    c = CASES[name]
    print(f"graph replay: {name}", flush=True)
    b = make_batch(c["ctx"], c["ql"], c["Hq"], c["Hkv"], c["D"])
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=b.num_q_heads, num_kv_heads=b.num_kv_heads,
                               head_dim=b.head_dim, block_size=b.block_size, dtype=b.dtype, device="cuda",
                               split_tokens=c["split"])
    eager = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table)
    torch.cuda.synchronize()
    assert_close_bf16(eager[: b.rows], oracle_paged(b), f"{name} eager")

    out = torch.empty_like(eager)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):                     # warm-up outside capture
        paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table, out=out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table, out=out)
    for rep in range(4):
        out.fill_(float("nan"))                       # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out[: b.rows].view(torch.int16), eager[: b.rows].view(torch.int16)), f"{name} replay {rep}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_whole_decode_step_graph(dtype):
    """One decode step of a config (a)-shaped model (16 layers, Llama-3.2-1B
    heads, block size 16, 8 sequences) as the layer loop of model.py:202-222
    runs it: per layer the RoPE + KV write and the paged attention
    (Attention.attention, attention.py:151-178), all 32 launches captured in
    one HIP graph.  Every replay (with eager work between) equals the eager
    step bit for bit in every layer's output and in the written cache."""
    import gllm_amd
    from oracle import metadata as om
    from oracle import rope as orope
    print(f"whole decode step graph {dtype}", flush=True)
    L, Hq, Hkv, D, bs, B = 16, 32, 8, 64, 16, 8
    g = torch.Generator().manual_seed(31)
    ctx = torch.randint(20, 200, (B,), generator=g).tolist()
    ql = [1] * B
    cache = gllm_amd.PagedKVCache(L, Hkv, D, bs, B, 256, dtype, "cuda")
    cache.physical_kv_cache.copy_(torch.randn(cache.physical_kv_cache.shape, generator=g).to(dtype))
    bt = om.random_block_tables([c + 1 for c in ctx], bs, cache.num_blocks, g, width=16)
    meta = om.build_metadata(ctx, ql, bt, bs, dtype)
    gm = gllm_amd.AttentionMetadata(
        query_lens=meta.query_lens.cuda(), seq_lens=meta.seq_lens.cuda(), max_seq_len=meta.max_seq_len,
        block_table=meta.block_table.cuda(), slot_mapping=meta.slot_mapping.cuda(),
        query_slot_mapping=meta.query_slot_mapping.cuda(), bias=None, block_size=bs)
    cos_t, sin_t = orope.rope_cache(256, D, 500000.0, dtype)
    pos = meta.positions
    cos, sin = cos_t[pos].cuda(), sin_t[pos].cuda()

    class Cfg:
        num_attn_heads, num_kv_heads, head_dim, hidden_size = Hq, Hkv, D, Hq * D

    Cfg.dtype = dtype
    w = lambda li: {f"model.layers.{li}.self_attn.{n}_proj.weight": torch.zeros(1) for n in "qkvo"}
    atts = [gllm_amd.Attention(li, Cfg, w(li)) for li in range(L)]
    qs = [torch.randn(B, 1, Hq, D, generator=g).to(dtype).cuda() for _ in range(L)]
    ks = [torch.randn(B, 1, Hkv, D, generator=g).to(dtype).cuda() for _ in range(L)]
    vs = [torch.randn(B, 1, Hkv, D, generator=g).to(dtype).cuda() for _ in range(L)]

    def step():
        return [atts[li].attention(qs[li], ks[li], vs[li], cos, sin, cache.get_layer_kv_cache(li), gm)
                for li in range(L)]

    eager = [o.clone() for o in step()]                  # also builds the plan, once for all layers
    cache_after = cache.physical_kv_cache.clone()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    bits = (lambda t: t.view(torch.int32)) if dtype == torch.float32 else (lambda t: t.view(torch.int16))
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))                        # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for li in range(L):
            assert torch.equal(bits(outs[li]), bits(eager[li])), f"replay {rep} layer {li}"
        assert torch.equal(cache.physical_kv_cache.view(torch.uint8), cache_after.view(torch.uint8))


@pytest.mark.parametrize("n", [16, 64, 700])
def test_qkv_projection_graph(n):
    """The fused QKV projection + RoPE + KV write (attention.py:139-161)
    captured in a HIP graph on each of its paths (16 tokens: one launch; 64:
    split-K partials + finish, with the cached workspace; 700: tile kernel):
    every replay, with eager work between, equals the eager call bit for bit
    in q and in the written cache."""
    from oracle import rope as orope
    print(f"qkv graph n={n}", flush=True)
    g = torch.Generator().manual_seed(200 + n)
    hidden, Hq, Hkv, D = 2048, 32, 8, 64
    bf = torch.bfloat16
    x = torch.randn(n, hidden, generator=g).to(bf).cuda()
    w = [(torch.randn(h * D, hidden, generator=g) / hidden ** 0.5).to(bf).cuda() for h in (Hq, Hkv, Hkv)]
    cos_t, sin_t = orope.rope_cache(4096, D, 500000.0, bf)
    cos_t, sin_t = cos_t.cuda(), sin_t.cuda()
    pos = torch.randint(0, 4096, (n,), generator=g).cuda()
    ns = 2 * n + 16
    slots = torch.randperm(ns, generator=g)[:n].cuda()
    kc = torch.zeros(ns, Hkv, D, dtype=bf, device="cuda")
    vc = torch.zeros_like(kc)
    q_out = torch.empty(n, Hq, D, dtype=bf, device="cuda")

    def call():
        paged.qkv_rope_kv_write(x, w[0], w[1], w[2], cos_t, sin_t, kc, vc, slots, q_out=q_out, rope_rows=pos,
                                unfused_from=None)

    call()
    torch.cuda.synchronize()
    q_eager, k_eager, v_eager = q_out.clone(), kc.clone(), vc.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for rep in range(4):
        q_out.fill_(float("nan"))                       # eager work between replays
        kc.zero_()
        vc.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(q_out.view(torch.int16), q_eager.view(torch.int16)), f"q replay {rep}"
        assert torch.equal(kc.view(torch.int16), k_eager.view(torch.int16)), f"k replay {rep}"
        assert torch.equal(vc.view(torch.int16), v_eager.view(torch.int16)), f"v replay {rep}"
