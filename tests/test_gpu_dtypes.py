"""Model and cache dtypes beyond bf16/bf16 (gllm/config/generator_params.py:9-10,
gllm/model/model.py:64,75: any torch dtype for the model and, separately, the
KV cache).  fp16 models run the MFMA kernels (fp16 MFMA, fp16 P); a 16-bit
model over an fp32 cache (or the other 16-bit type) runs the generic kernel,
which casts each cached value to the model dtype as the reference's gather
does (attention.py:169-170).  Bar: the RoPE + KV write bit-exact against the
oracle's per-op restatement; attention outputs within max-abs 2e-2 /
mean-abs 2e-3 of the fp32 oracle (the benchmark bar, also used for fp16)."""
import pytest
import torch

import gllm_amd
from gllm_amd import paged, workloads
from oracle import attention as oa
from oracle import metadata as om
from oracle import rope as orope
from tests.gpu_helpers import assert_close_bf16, oracle_paged

pytestmark = pytest.mark.gpu
DEV = "cuda"
F16, BF, F32, F8 = torch.float16, torch.bfloat16, torch.float32, torch.float8_e4m3fn


def _bits(t):
    t = t.cpu().contiguous()
    return t.view({1: torch.uint8, 2: torch.int16, 4: torch.int32}[t.element_size()])


def _batch(ctx, ql, Hq, Hkv, D, dtype, kv_dtype=None, bs=16, fresh_cache=False, theta=None, seed=2):
    seq = [c + q for c, q in zip(ctx, ql)]
    nb = sum(-(-L // bs) for L in seq) * 2 + 8
    b = workloads.PagedBatch("t", list(ctx), list(ql), Hq, Hkv, D, bs, nb, dtype, rope_theta=theta,
                             kv_dtype=kv_dtype)
    b = workloads.materialize(b, DEV, seed=seed)
    if fresh_cache:   # values the model dtype cannot hold, so the gather's cast is exercised
        g = torch.Generator().manual_seed(seed + 100)
        b.k_cache = torch.randn(b.k_cache.shape, generator=g).to(kv_dtype).to(DEV)
        b.v_cache = torch.randn(b.v_cache.shape, generator=g).to(kv_dtype).to(DEV)
    return b


# ------------------------------------------------------------ RoPE + KV write
@pytest.mark.parametrize("dtype,kv_dtype,D", [(F16, F16, 64), (F16, F16, 128), (F16, F8, 128), (F16, F32, 64),
                                              (F16, BF, 128), (BF, F32, 128), (BF, F16, 64), (F32, F16, 64)])
def test_rope_kv_write_bit_exact_any_pairing(dtype, kv_dtype, D):
    """attention.py:151-161 with model dtype != bf16 or a cache of another
    dtype: every op rounded to the model dtype, the written rows cast like
    torch's .to(kv_dtype) (bit-exact, sentinel pool untouched elsewhere)."""
    print(f"rope_kv_write {dtype} -> {kv_dtype} D={D}", flush=True)
    g = torch.Generator().manual_seed(40 + D)
    ctx, ql = [0, 17, 40, 3], [9, 1, 24, 16]
    Hq, Hkv, bs, nb = 8, 2, 16, 64
    bt = om.random_block_tables([c + q for c, q in zip(ctx, ql)], bs, nb, g, width=8)
    meta = om.build_metadata(ctx, ql, bt, bs, dtype)
    B, Tq = meta.query_slot_mapping.shape
    q = (torch.randn(B, Tq, Hq, D, generator=g) * 4).to(dtype)
    k = (torch.randn(B, Tq, Hkv, D, generator=g) * 4).to(dtype)
    v = (torch.randn(B, Tq, Hkv, D, generator=g) * 4).to(dtype)
    cos_t, sin_t = orope.rope_cache(128, D, 500000.0, dtype)
    cos, sin = cos_t[meta.positions], sin_t[meta.positions]
    sk = torch.randn(nb * bs, Hkv, D, generator=g).to(kv_dtype)
    sv = torch.randn(nb * bs, Hkv, D, generator=g).to(kv_dtype)
    kc_ref, vc_ref = sk.clone(), sv.clone()
    q_ref = orope.apply_rope(q, cos, sin)
    oa.kv_write(kc_ref, vc_ref, meta.query_slot_mapping, orope.apply_rope(k, cos, sin), v)
    kc, vc = sk.to(DEV), sv.to(DEV)
    q_out = torch.full((B, Tq, Hq, D), 7.0, dtype=dtype, device=DEV)
    paged.rope_kv_write(k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV), kc, vc, meta.query_slot_mapping.to(DEV),
                        query_lens=meta.query_lens.to(DEV), q=q.to(DEV), q_out=q_out)
    torch.cuda.synchronize()
    # block 0 is the dummy the reference's padded rows write (the kernel skips them)
    assert torch.equal(_bits(kc)[bs:], _bits(kc_ref)[bs:])
    assert torch.equal(_bits(vc)[bs:], _bits(vc_ref)[bs:])
    assert torch.equal(_bits(kc)[:bs], _bits(sk)[:bs])
    for i in range(B):
        assert torch.equal(_bits(q_out[i, :ql[i]]), _bits(q_ref[i, :ql[i]]))


# ------------------------------------------------------------ fp16 model on the MFMA kernels
@pytest.mark.parametrize("kv", [F16, F8])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("split", [0, 256, paged.BALANCED])
def test_fp16_decode(kv, D, split):
    print(f"fp16 decode kv={kv} D={D} split={split}", flush=True)
    b = _batch([300, 1000, 17, 4000, 64, 2047], [1] * 6, 32, 8, D, F16, kv)
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=32, num_kv_heads=8, head_dim=D, block_size=16,
                               dtype=F16, device=DEV, split_tokens=split)
    out = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table)
    torch.cuda.synchronize()
    assert out.dtype == F16
    assert_close_bf16(out, oracle_paged(b), "fp16 decode")


@pytest.mark.parametrize("kv", [F16, F8])
@pytest.mark.parametrize("D", [64, 128])
def test_fp16_prefill_and_mixed(kv, D):
    """Prefill items alone (RoPE on load) and a mixed launch of decode rows
    and prefill chunks, fp16 model."""
    print(f"fp16 prefill/mixed kv={kv} D={D}", flush=True)
    b = _batch([0, 0, 37, 300], [33, 130, 77, 45], 32, 8, D, F16, kv, theta=500000.0)
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=32, num_kv_heads=8, head_dim=D, block_size=16,
                               dtype=F16, device=DEV)
    out = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table, rope=(b.cos, b.sin, "position"))
    torch.cuda.synchronize()
    pos = torch.cat([torch.arange(c, c + q) for c, q in zip(b.ctx_lens, b.q_lens)])
    qr = orope.apply_rope(b.q.cpu().unsqueeze(0), b.cos.cpu()[pos].unsqueeze(0), b.sin.cpu()[pos].unsqueeze(0))[0]
    assert_close_bf16(out, oracle_paged(b, qr), "fp16 prefill")
    m = _batch([300, 0, 57, 1000, 5, 2500], [1, 120, 64, 1, 1, 1], 32, 8, D, F16, kv)
    plan = paged.AttentionPlan(m.q_lens, m.seq_lens, num_q_heads=32, num_kv_heads=8, head_dim=D, block_size=16,
                               dtype=F16, device=DEV)
    out = paged.paged_attention(plan, m.q, m.k_cache, m.v_cache, m.block_table)
    torch.cuda.synchronize()
    assert_close_bf16(out, oracle_paged(m), "fp16 mixed")


@pytest.mark.parametrize("D", [64, 128])
def test_fp16_prefill_extreme_scores(D):
    """fp16 P holds at most 65504: the prefill softmax keeps p <= 2^15 (row
    reference from the first half-tile's max, fix-up past 2^15).  Scores far
    beyond that range (q x 30), against the unmodified fp32 oracle."""
    print(f"fp16 extreme scores D={D}", flush=True)
    b = _batch([0, 0, 100], [200, 70, 90], 32, 8, D, F16)
    b.q.mul_(30.0)
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=32, num_kv_heads=8, head_dim=D, block_size=16,
                               dtype=F16, device=DEV)
    out = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table)
    torch.cuda.synchronize()
    assert_close_bf16(out, oracle_paged(b), "fp16 prefill, scaled q")


@pytest.mark.parametrize("B,Tq,T,Hq,Hkv,D", [(1, 40, 40, 1, 1, 128), (3, 5, 77, 32, 8, 64), (2, 96, 160, 8, 2, 128),
                                             (1, 17, 33, 4, 2, 80)])
def test_fp16_dense_op(B, Tq, T, Hq, Hkv, D):
    """reference_attention(q, k, v, bias) in fp16 (the MFMA kernel at D 64 /
    128, the generic kernel otherwise), causal-with-offset bias."""
    print(f"fp16 dense {B},{Tq},{T},{Hq},{Hkv},{D}", flush=True)
    g = torch.Generator().manual_seed(B * 100 + T)
    q = torch.randn(B, Tq, Hq, D, generator=g).to(F16)
    k = torch.randn(B, T, Hkv, D, generator=g).to(F16)
    v = torch.randn(B, T, Hkv, D, generator=g).to(F16)
    bias = torch.zeros(B, Tq, T, dtype=F16)
    bias[:, :, T - Tq:] = torch.full((Tq, Tq), float("-inf")).triu(1).to(F16)
    ref = oa.reference_attention(q.float(), k.float(), v.float(), bias.float())
    out = gllm_amd.reference_attention(q.to(DEV), k.to(DEV), v.to(DEV), bias.to(DEV))
    torch.cuda.synchronize()
    assert out.dtype == F16
    assert_close_bf16(out, ref, "fp16 dense")


def test_fp16_generic_head_dim():
    """An fp16 model with a head dim the MFMA kernels do not take (80): the
    generic kernel, decode and prefill rows in one batch."""
    print("fp16 generic D=80", flush=True)
    b = _batch([100, 0, 20], [1, 40, 9], 8, 2, 80, F16)
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=8, num_kv_heads=2, head_dim=80, block_size=16,
                               dtype=F16, device=DEV)
    out = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table)
    torch.cuda.synchronize()
    assert_close_bf16(out, oracle_paged(b), "fp16 generic")


# ------------------------------------------------------------ 16-bit model over another cache dtype
@pytest.mark.parametrize("model,cache", [(BF, F32), (F16, F32), (BF, F16), (F16, BF)])
@pytest.mark.parametrize("D", [64, 128])
def test_model_over_other_cache_dtype(model, cache, D):
    """The cache holds values the model dtype cannot (fresh fp32 draws, or
    the other 16-bit type): each is rounded to the model dtype on read, as
    the reference's gather casts it; decode and prefill rows in one batch."""
    print(f"model {model} over cache {cache} D={D}", flush=True)
    b = _batch([300, 0, 57, 1000, 5], [1, 70, 64, 1, 1], 32, 8, D, model, cache, fresh_cache=True)
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=32, num_kv_heads=8, head_dim=D, block_size=16,
                               dtype=model, device=DEV)
    out = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table)
    torch.cuda.synchronize()
    assert out.dtype == model
    ref = oracle_paged(b)                         # gathers with .to(q.dtype), then fp32
    assert_close_bf16(out, ref, f"{model} over {cache}")
    # the cast matters: the same attention over the unrounded cache differs
    raw = oa.paged_attention(b.q.cpu().float(), b.k_cache.cpu().float(), b.v_cache.cpu().float(),
                             b.block_table.cpu(), b.ctx_lens, b.q_lens, b.q_row_start, 16)
    if cache == F32 or (model == BF and cache == F16):
        assert (ref - raw).abs().max().item() > 1e-4


@pytest.mark.parametrize("dtype", [BF, F16])
@pytest.mark.parametrize("kv,D", [(None, 64), (None, 128), (F8, 64), (F8, 128)])
def test_rope_on_load_bit_identical(dtype, kv, D):
    """q rotated inside the attention kernels (decode and prefill items, the
    fp8 / D = 64 decode path rotating half a pair per lane included) gives
    the same output bits as attention over q rotated first by the RoPE
    kernel (itself bit-exact against apply_rope)."""
    print(f"rope on load {dtype} kv={kv} D={D}", flush=True)
    b = _batch([10, 500, 0, 37], [1, 1, 70, 40], 32, 8, D, dtype, kv, theta=500000.0)
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=32, num_kv_heads=8, head_dim=D, block_size=16,
                               dtype=dtype, device=DEV)
    pos = torch.cat([torch.arange(c, c + q) for c, q in zip(b.ctx_lens, b.q_lens)]).to(DEV)
    out1 = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table, rope=(b.cos, b.sin, "position"))
    qr = paged.rope_rotate(b.q, b.cos, b.sin, rope_rows=pos)
    out2 = paged.paged_attention(plan, qr, b.k_cache, b.v_cache, b.block_table)
    torch.cuda.synchronize()
    assert torch.equal(_bits(out1), _bits(out2))
