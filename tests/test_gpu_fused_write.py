"""The decode step's RoPE + KV write folded into the attention launch
(gllm_paged_attention_write_kv; gllm/model/layers/attention.py:151-178 as one
launch per layer) against the two-call sequence it replaces: gllm_rope_kv_write
through the reference's query_slot_mapping, then gllm_paged_attention.  On
the MFMA kernels the attention reads the written keys back from the cache,
so outputs and caches are bit-identical; the generic kernel keeps the new
keys in LDS (the same values) and sums them in another order, so its output
agrees to fp32 rounding and the cache bit for bit.  Both are also checked
against the fp32 oracle."""
import pytest
import torch

from gllm_amd import paged, workloads
from tests.gpu_helpers import assert_close_bf16, oracle_paged

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bits(t):
    t = t.cpu().contiguous()
    return t.view({1: torch.uint8, 2: torch.int16, 4: torch.int32}[t.element_size()])


def _case(ctx, ql, Hq, Hkv, D, dtype, kv_dtype=None, split=0, bs=16, rope="row", seed=3):
    seq = [c + q for c, q in zip(ctx, ql)]
    nb = sum(-(-L // bs) for L in seq) * 2 + 8
    b = workloads.PagedBatch("f", list(ctx), list(ql), Hq, Hkv, D, bs, nb, dtype, rope_theta=500000.0,
                             kv_dtype=kv_dtype)
    b = workloads.materialize(b, DEV, seed=seed)
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=Hq, num_kv_heads=Hkv, head_dim=D, block_size=bs,
                               dtype=dtype, device=DEV, split_tokens=split)
    pos = torch.cat([torch.arange(c, c + q) for c, q in zip(b.ctx_lens, b.q_lens)]).to(DEV)
    if rope == "row":     # one cos/sin row per query row (Attention.attention's cos_pos)
        cs, sn, rr = b.cos[pos].contiguous(), b.sin[pos].contiguous(), None
    else:                 # the table, rows c_i + r
        cs, sn, rr = b.cos, b.sin, pos
    return b, plan, cs, sn, rr


def _run_both(b, plan, cs, sn, rr, rope):
    kc1, vc1 = b.k_cache.clone(), b.v_cache.clone()
    kc2, vc2 = b.k_cache.clone(), b.v_cache.clone()
    # two calls: the write through the slot mapping, then the attention
    paged.rope_kv_write(b.k_new, b.v_new, cs, sn, kc1, vc1, b.slot_mapping, rope_rows=rr)
    o1 = paged.paged_attention(plan, b.q, kc1, vc1, b.block_table, rope=(cs, sn, rope))
    # one launch
    assert paged.fused_kv_write_ok(plan, kc2.dtype)
    o2 = paged.paged_attention(plan, b.q, kc2, vc2, b.block_table, rope=(cs, sn, rope), kv_new=(b.k_new, b.v_new))
    torch.cuda.synchronize()
    return o1, o2, (kc1, vc1), (kc2, vc2)


def _oracle(b, cs, sn, rope, caches):
    from oracle import rope as orope
    pos = torch.cat([torch.arange(c, c + q) for c, q in zip(b.ctx_lens, b.q_lens)])
    c = cs.cpu() if rope == "row" else cs.cpu()[pos]
    s = sn.cpu() if rope == "row" else sn.cpu()[pos]
    qr = orope.apply_rope(b.q.cpu().unsqueeze(0), c.unsqueeze(0), s.unsqueeze(0))[0]
    b.k_cache, b.v_cache = caches
    return oracle_paged(b, qr)


@pytest.mark.parametrize("dtype,kv,D,split", [(torch.bfloat16, None, 64, 0), (torch.bfloat16, None, 128, 0),
                                              (torch.bfloat16, None, 128, 256), (torch.bfloat16, None, 64, -1),
                                              (torch.bfloat16, torch.float8_e4m3fn, 64, 0),
                                              (torch.bfloat16, torch.float8_e4m3fn, 128, -1),
                                              (torch.float16, None, 128, 0), (torch.float16, None, 64, 256)])
@pytest.mark.parametrize("rope", ["row", "position"])
def test_fused_write_mfma_bit_exact(dtype, kv, D, split, rope):
    """Split and page-balanced plans (the new key sits in a sequence's last
    split / segment), fp8 caches, fp16 models: output and cache bit-exact
    against the two calls."""
    print(f"fused write mfma {dtype} kv={kv} D={D} split={split} rope={rope}", flush=True)
    split = paged.BALANCED if split == -1 else split
    b, plan, cs, sn, rr = _case([40, 700, 0, 2500, 15, 1023], [1] * 6, 32, 8, D, dtype, kv, split=split,
                                rope=rope)
    o1, o2, c1, c2 = _run_both(b, plan, cs, sn, rr, rope)
    assert torch.equal(_bits(c1[0]), _bits(c2[0])) and torch.equal(_bits(c1[1]), _bits(c2[1]))
    assert torch.equal(_bits(o1), _bits(o2))
    assert_close_bf16(o2, _oracle(b, cs, sn, rope, c2), "fused")


def test_fused_write_multi_row_decode():
    """Decode-path sequences with several query rows (q_len x G <= 16, G = 4):
    several new keys per sequence, each visible from its own row on."""
    print("fused write multi-row decode", flush=True)
    b, plan, cs, sn, rr = _case([33, 0, 300, 17], [4, 2, 3, 1], 32, 8, 128, torch.bfloat16)
    assert plan.info["prefill_seqs"] == 0
    o1, o2, c1, c2 = _run_both(b, plan, cs, sn, rr, "row")
    assert torch.equal(_bits(c1[0]), _bits(c2[0])) and torch.equal(_bits(c1[1]), _bits(c2[1]))
    assert torch.equal(_bits(o1), _bits(o2))


@pytest.mark.parametrize("dtype,kv,D", [(torch.float32, None, 64), (torch.float32, torch.bfloat16, 64),
                                        (torch.bfloat16, torch.float32, 128), (torch.bfloat16, None, 80),
                                        (torch.float32, None, 96)])
def test_fused_write_generic_kernel(dtype, kv, D):
    """fp32 models (config (a)), a 16-bit model over an fp32 cache, odd head
    dims: the generic kernel's fused path, single- and multi-row decode."""
    print(f"fused write generic {dtype} kv={kv} D={D}", flush=True)
    b, plan, cs, sn, rr = _case([40, 200, 0, 97], [1, 3, 1, 16], 8, 2, D, dtype, kv)
    o1, o2, c1, c2 = _run_both(b, plan, cs, sn, rr, "row")
    assert torch.equal(_bits(c1[0]), _bits(c2[0])) and torch.equal(_bits(c1[1]), _bits(c2[1]))
    d = (o1.float() - o2.float()).abs().max().item()
    assert d < (2e-6 if dtype == torch.float32 else 1e-2), d
    if dtype == torch.float32:
        ref = _oracle(b, cs, sn, "row", c2)
        assert (o2.cpu() - ref).abs().max().item() < 1e-4
    else:
        assert_close_bf16(o2, _oracle(b, cs, sn, "row", c2), "fused generic")


def test_fused_write_rejects_prefill_plans():
    print("fused write rejects prefill plans", flush=True)
    b, plan, cs, sn, rr = _case([0, 40], [100, 1], 32, 8, 128, torch.bfloat16)
    assert not paged.fused_kv_write_ok(plan, b.k_cache.dtype)
    with pytest.raises(ValueError, match="decode-path"):
        paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table, rope=(cs, sn, "row"),
                              kv_new=(b.k_new, b.v_new))


@pytest.mark.parametrize("bs", [1, 7, 64])
@pytest.mark.parametrize("dtype,kv,D", [(torch.bfloat16, None, 128), (torch.bfloat16, torch.float8_e4m3fn, 64),
                                        (torch.float32, None, 64)])
def test_fused_write_block_sizes(bs, dtype, kv, D):
    """Block sizes other than 16 (the slot comes from the block table at key
    position c_i + r through the plan's block-size division): output and
    cache against the two calls, on the MFMA and the generic kernel."""
    print(f"fused write bs={bs} {dtype} kv={kv} D={D}", flush=True)
    b, plan, cs, sn, rr = _case([40, 700, 0, 130, 15], [1, 1, 1, 2, 1], 32, 8, D, dtype, kv, bs=bs)
    o1, o2, c1, c2 = _run_both(b, plan, cs, sn, rr, "row")
    assert torch.equal(_bits(c1[0]), _bits(c2[0])) and torch.equal(_bits(c1[1]), _bits(c2[1]))
    if dtype == torch.float32:
        assert (o1 - o2).abs().max().item() < 2e-6
    else:
        assert torch.equal(_bits(o1), _bits(o2))


def test_fused_write_in_attention_forward_graph():
    """gllm_amd.Attention on a decode step takes the fused path; the step
    captured in a HIP graph and replayed matches eager bit for bit (outputs
    and the written cache)."""
    import gllm_amd
    print("fused write attention graph", flush=True)
    L, Hq, Hkv, D, bs, B = 2, 32, 8, 64, 16, 4
    ctx = [30, 200, 5, 77]
    seq = [c + 1 for c in ctx]
    cache = gllm_amd.PagedKVCache(L, Hkv, D, bs, B, 256, torch.bfloat16, DEV)
    cache.physical_kv_cache.normal_()
    bt = workloads.block_tables(seq, bs, cache.num_blocks).to(DEV)
    pos = torch.tensor(ctx)
    qsm = (bt.cpu()[torch.arange(B), pos // bs].to(torch.int64) * bs + pos % bs).view(B, 1).to(DEV)
    meta = gllm_amd.AttentionMetadata(query_lens=torch.ones(B, dtype=torch.int32, device=DEV),
                                      seq_lens=torch.tensor(seq, dtype=torch.int32, device=DEV), max_seq_len=max(seq),
                                      block_table=bt, slot_mapping=None, query_slot_mapping=qsm, bias=None,
                                      block_size=bs)
    ang = pos.unsqueeze(1) * 500000.0 ** (-2 * torch.arange(D // 2) / D)
    cos = torch.cos(ang).to(torch.bfloat16).view(B, 1, -1).to(DEV)
    sin = torch.sin(ang).to(torch.bfloat16).view(B, 1, -1).to(DEV)

    class Cfg:
        num_attn_heads, num_kv_heads, head_dim, hidden_size, dtype = Hq, Hkv, D, Hq * D, torch.bfloat16

    atts = [gllm_amd.Attention(li, Cfg, {f"model.layers.{li}.self_attn.{n}_proj.weight": torch.zeros(1)
                                         for n in "qkvo"}) for li in range(L)]
    g = torch.Generator(device=DEV).manual_seed(5)
    qs = [torch.randn(B, 1, Hq, D, device=DEV, generator=g).to(torch.bfloat16) for _ in range(L)]
    ks = [torch.randn(B, 1, Hkv, D, device=DEV, generator=g).to(torch.bfloat16) for _ in range(L)]
    vs = [torch.randn(B, 1, Hkv, D, device=DEV, generator=g).to(torch.bfloat16) for _ in range(L)]
    pristine = cache.physical_kv_cache.clone()

    def step():
        return [atts[li].attention(qs[li], ks[li], vs[li], cos, sin, cache.get_layer_kv_cache(li), meta)
                for li in range(L)]

    eager = [o.clone() for o in step()]
    torch.cuda.synchronize()
    assert paged.fused_kv_write_ok(meta._gllm_plan, torch.bfloat16)
    eager_cache = cache.physical_kv_cache.clone()
    cache.physical_kv_cache.copy_(pristine)
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()                                    # warm up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        outs = step()
    for _ in range(3):
        cache.physical_kv_cache.copy_(pristine)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(_bits(o), _bits(e))
        assert torch.equal(_bits(cache.physical_kv_cache), _bits(eager_cache))
