"""GPU parity of the HIP kernels against the CPU oracle (identical seeded
inputs).  Bar: bit-exact for the RoPE/KV-write indexing and values; bf16
attention outputs within max-abs 2e-2 and mean-abs 2e-3 of the fp32 oracle;
fp32 outputs within 1e-4."""

import pytest
import torch

import gllm_amd
from gllm_amd import paged
from oracle import attention as oa
from oracle import metadata as om
from oracle import rope as orope
from tests.gpu_helpers import assert_close_bf16, make_batch, oracle_paged

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bits(t):
    return t.cpu().contiguous().view({1: torch.uint8, 2: torch.int16, 4: torch.int32}[t.element_size()])


# ------------------------------------------------------------ (a) RoPE + KV write
@pytest.mark.parametrize("dtype,kv_dtype,D", [(torch.bfloat16, torch.bfloat16, 64),
                                              (torch.bfloat16, torch.bfloat16, 128),
                                              (torch.float32, torch.float32, 64),
                                              (torch.float32, torch.bfloat16, 128),
                                              # fp8 cache: the write must round like torch's .to(float8_e4m3fn)
                                              (torch.bfloat16, torch.float8_e4m3fn, 64),
                                              (torch.bfloat16, torch.float8_e4m3fn, 128),
                                              (torch.float32, torch.float8_e4m3fn, 64)])
def test_rope_kv_write_bit_exact(dtype, kv_dtype, D):
    print(f"rope_kv_write dtype={dtype} kv={kv_dtype} D={D}", flush=True)
    g = torch.Generator().manual_seed(10 + D)
    ctx = [0, 17, 40, 3]
    ql = [9, 1, 24, 16]
    Hq, Hkv, bs, nb = 8, 2, 16, 64
    bt = om.random_block_tables([c + q for c, q in zip(ctx, ql)], bs, nb, g, width=8)
    meta = om.build_metadata(ctx, ql, bt, bs, dtype)
    B, Tq = meta.query_slot_mapping.shape
    q = torch.randn(B, Tq, Hq, D, generator=g).to(dtype)
    k = torch.randn(B, Tq, Hkv, D, generator=g).to(dtype)
    v = torch.randn(B, Tq, Hkv, D, generator=g).to(dtype)
    cos_t, sin_t = orope.rope_cache(128, D, 500000.0, dtype)
    cos, sin = cos_t[meta.positions], sin_t[meta.positions]
    sentinel_k = torch.randn(nb * bs, Hkv, D, generator=g).to(kv_dtype)
    sentinel_v = torch.randn(nb * bs, Hkv, D, generator=g).to(kv_dtype)
    # oracle: reference order (attention.py:151-161) on CPU
    kc_ref, vc_ref = sentinel_k.clone(), sentinel_v.clone()
    q_ref = orope.apply_rope(q, cos, sin)
    k_ref = orope.apply_rope(k, cos, sin)
    oa.kv_write(kc_ref, vc_ref, meta.query_slot_mapping, k_ref, v)
    # product
    kc, vc = sentinel_k.to(DEV), sentinel_v.to(DEV)
    q_out = torch.full((B, Tq, Hq, D), 7.0, dtype=dtype, device=DEV)
    paged.rope_kv_write(k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV), kc, vc,
                        meta.query_slot_mapping.to(DEV), query_lens=meta.query_lens.to(DEV),
                        q=q.to(DEV), q_out=q_out)
    torch.cuda.synchronize()
    # block 0 is the dummy the reference's padded rows write; everything else bit-exact
    assert torch.equal(_bits(kc)[bs:], _bits(kc_ref)[bs:])
    assert torch.equal(_bits(vc)[bs:], _bits(vc_ref)[bs:])
    assert torch.equal(_bits(kc)[:bs], _bits(sentinel_k)[:bs])  # padded rows skipped
    for i in range(B):
        assert torch.equal(_bits(q_out[i, :ql[i]]), _bits(q_ref[i, :ql[i]]))
        assert bool((q_out[i, ql[i]:] == 7.0).all())   # padded rows: not written, cos/sin not read
    # apply_rope drop-in on a whole tensor
    qr = paged.rope_rotate(q.to(DEV), cos.to(DEV), sin.to(DEV))
    assert torch.equal(_bits(qr), _bits(q_ref))


def test_fp8_cache_cast_exhaustive():
    """Every bf16 bit pattern (NaN, inf, subnormals, overflow included) and a
    set of fp32 values written to an fp8 cache through the V path: bytes equal
    torch's .to(float8_e4m3fn) (the reference's write, attention.py:161)."""
    Hkv, D = 1, 64
    allb = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).reshape(-1, Hkv, D)
    g = torch.Generator().manual_seed(77)
    f32 = torch.cat([torch.randn(59968, generator=g) * 300, torch.tensor(
        [464.0, 463.99, 464.01, 448.0, 480.0, -464.0, 2 ** -10, 3 * 2 ** -10, 2 ** -6, 2 ** -6 * 0.999,
         float("inf"), float("-inf"), float("nan"), -float("nan"), 0.0, -0.0] * 4)]).reshape(-1, Hkv, D)
    for v in (allb, f32):
        n = v.shape[0]
        k = torch.zeros_like(v)
        cos = torch.ones(n, D // 2, dtype=v.dtype)
        sin = torch.zeros(n, D // 2, dtype=v.dtype)
        kc = torch.zeros(n, Hkv, D, dtype=torch.float8_e4m3fn, device=DEV)
        vc = torch.zeros(n, Hkv, D, dtype=torch.float8_e4m3fn, device=DEV)
        slots = torch.arange(n, dtype=torch.int64)
        paged.rope_kv_write(k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV), kc, vc, slots.to(DEV))
        torch.cuda.synchronize()
        assert torch.equal(vc.cpu().view(torch.uint8), v.to(torch.float8_e4m3fn).view(torch.uint8)), v.dtype


# ------------------------------------------------------------ (b) decode
@pytest.mark.parametrize("Hq,Hkv,D", [(32, 8, 64), (32, 8, 128), (64, 8, 128), (8, 8, 64), (16, 1, 64)])
@pytest.mark.parametrize("split", [0, 32, 96, paged.BALANCED])
def test_decode_parity(Hq, Hkv, D, split):
    print(f"decode Hq={Hq} Hkv={Hkv} D={D} split={split}", flush=True)
    lens = [1, 2, 15, 16, 17, 31, 32, 33, 63, 64, 65, 100, 255, 256, 257, 700, 1025]
    b = make_batch([L - 1 for L in lens], [1] * len(lens), Hq, Hkv, D)
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=Hq, num_kv_heads=Hkv, head_dim=D,
                               block_size=16, dtype=torch.bfloat16, device=DEV, split_tokens=split)
    ref = oracle_paged(b)
    for rep in range(2):  # second launch checks the split tickets were reset
        out = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table)
        torch.cuda.synchronize()
        assert_close_bf16(out, ref, f"decode rep {rep}")


@pytest.mark.parametrize("split", [0, 64, paged.BALANCED])
def test_decode_multi_query_rows(split):
    """q_len * G <= 16 stays on the decode path with a causal mask inside it
    (page-balanced: a segment past a row's last visible key leaves that row's
    partial empty)."""
    print(f"decode multi-query split={split}", flush=True)
    b = make_batch([40, 0, 200, 7, 1000], [4, 3, 2, 4, 4], 16, 4, 64)
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=16, num_kv_heads=4, head_dim=64,
                               block_size=16, dtype=torch.bfloat16, device=DEV, split_tokens=split)
    assert plan.info["decode_seqs"] == 5
    for rep in range(2):
        out = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table)
        torch.cuda.synchronize()
        assert_close_bf16(out, oracle_paged(b), f"decode multi-row rep {rep}")


@pytest.mark.parametrize("bs", [4, 8, 32, 64])
@pytest.mark.parametrize("Hq,Hkv,D", [(16, 2, 64), (32, 4, 128), (48, 12, 64)])
def test_decode_balanced_shapes(bs, Hq, Hkv, D):
    """Page-balanced decode over block sizes (segment cuts at 16-key units,
    not block boundaries) and kv-head groupings (Hkv 2 / 4 -> 2 / 4 heads
    per workgroup, Hkv 12 -> three groups of 4)."""
    print(f"decode balanced bs={bs} Hq={Hq} Hkv={Hkv} D={D}", flush=True)
    lens = [1, 9, 16, 47, 130, 511, 2100, 3000]
    b = make_batch([L - 1 for L in lens], [1] * len(lens), Hq, Hkv, D, bs=bs)
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=Hq, num_kv_heads=Hkv, head_dim=D,
                               block_size=bs, dtype=torch.bfloat16, device=DEV, split_tokens=paged.BALANCED)
    info = plan.info
    assert info["decode_segments"] > 0 and info["heads_per_wg"] == (2 if Hkv == 2 else 4)
    ref = oracle_paged(b)
    for rep in range(2):
        out = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table)
        torch.cuda.synchronize()
        assert_close_bf16(out, ref, f"balanced rep {rep}")


# ------------------------------------------------------------ (c) prefill
@pytest.mark.parametrize("Hq,Hkv,D", [(32, 8, 128), (32, 8, 64), (8, 1, 64), (16, 16, 128), (64, 8, 128)])
def test_prefill_parity(Hq, Hkv, D):
    print(f"prefill Hq={Hq} Hkv={Hkv} D={D}", flush=True)
    ctx = [0, 0, 0, 37, 300]
    ql = [1 + 32, 130, 64, 77, 45]
    b = make_batch(ctx, ql, Hq, Hkv, D)
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=Hq, num_kv_heads=Hkv, head_dim=D,
                               block_size=16, dtype=torch.bfloat16, device=DEV)
    out = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table)
    torch.cuda.synchronize()
    assert_close_bf16(out, oracle_paged(b), "prefill")


@pytest.mark.parametrize("D", [64, 128])
def test_prefill_extreme_scores(D):
    """Scores far outside the softmax fast path's range [-64, 64] (log2
    units), against the unmodified fp32 oracle at the usual bar: q scaled up
    (most half-tiles overflow 2^64 and take the fix-up), and a first
    half-tile far below every later key (the row's reference starts at that
    max, later tiles move it up).  The kernel scales the fp32 scores, so
    large logits cost no precision; a wrong rescale would be off by O(1)."""
    print(f"prefill extreme scores D={D}", flush=True)
    Hq, Hkv = 32, 8
    b = make_batch([0, 0, 100], [200, 70, 90], Hq, Hkv, D)
    b.q.mul_(30.0)                                          # s ~ N(0, (30 * 1.44)^2): row maxima > 64
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=Hq, num_kv_heads=Hkv, head_dim=D,
                               block_size=16, dtype=torch.bfloat16, device=DEV)
    out = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table)
    torch.cuda.synchronize()
    assert_close_bf16(out, oracle_paged(b), "prefill, scaled q")
    # every query row = u; keys 0..31 of each sequence = -6 u / |u| * sqrt(D): first half-tile
    # scores ~ -6 sqrt(D) * 1.44 < -64, later keys N(0, 1) scores
    g = torch.Generator().manual_seed(7)
    c = make_batch([0, 40], [100, 60], Hq, Hkv, D)
    u = torch.randn(D, generator=g)
    u = u / u.norm() * D ** 0.5
    c.q.copy_(u.to(c.q.dtype).expand_as(c.q))
    bt = c.block_table.cpu()
    for i in range(2):
        for p in range(32):
            slot = int(bt[i, p // 16]) * 16 + p % 16
            c.k_cache[slot] = (-6.0 * u).to(c.k_cache.dtype).to(DEV)
    plan = paged.AttentionPlan(c.q_lens, c.seq_lens, num_q_heads=Hq, num_kv_heads=Hkv, head_dim=D,
                               block_size=16, dtype=torch.bfloat16, device=DEV)
    out = paged.paged_attention(plan, c.q, c.k_cache, c.v_cache, c.block_table)
    torch.cuda.synchronize()
    assert_close_bf16(out, oracle_paged(c), "prefill, very negative first tile")


@pytest.mark.parametrize("scale", [10.0, 30.0])
def test_mixed_extreme_scores(scale):
    """A mixed launch (decode rows and prefill chunks in one grid) with q
    scaled up, against the unmodified fp32 oracle: both item kinds scale
    their fp32 scores."""
    print(f"mixed extreme scores x{scale}", flush=True)
    b = make_batch([300, 0, 57, 1000, 5], [1, 120, 64, 1, 1], 32, 8, 128)
    b.q.mul_(scale)
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=32, num_kv_heads=8, head_dim=128,
                               block_size=16, dtype=torch.bfloat16, device=DEV)
    out = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table)
    torch.cuda.synchronize()
    assert_close_bf16(out, oracle_paged(b), "mixed, scaled q")


@pytest.mark.parametrize("D", [64, 128])
def test_dense_op_extreme_scores(D):
    """The dense-bias op (reference_attention contract) with logits far
    beyond N(0,1): q scaled by 30, engine-style causal bias, against the
    fp32 op on the same bf16 inputs."""
    print(f"dense extreme scores D={D}", flush=True)
    g = torch.Generator().manual_seed(70 + D)
    B, Tq, T, Hq, Hkv = 2, 96, 160, 8, 2
    q = (torch.randn(B, Tq, Hq, D, generator=g) * 30.0).to(torch.bfloat16)
    k = torch.randn(B, T, Hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, T, Hkv, D, generator=g).to(torch.bfloat16)
    bias = torch.zeros(B, Tq, T, dtype=torch.bfloat16)
    bias[:, :, T - Tq:] = torch.full((Tq, Tq), float("-inf")).triu(1).to(torch.bfloat16)
    ref = oa.reference_attention(q.float(), k.float(), v.float(), bias.float())
    out = gllm_amd.reference_attention(q.to(DEV), k.to(DEV), v.to(DEV), bias.to(DEV))
    torch.cuda.synchronize()
    assert_close_bf16(out, ref, "dense, scaled q")


def test_prefill_rope_in_kernel_matches_prerotated():
    """RoPE fused into the attention kernel's q load == RoPE applied first."""
    print("prefill rope fused", flush=True)
    b = make_batch([0, 50], [100, 70], 32, 8, 128, theta=500000.0)
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=32, num_kv_heads=8, head_dim=128,
                               block_size=16, dtype=torch.bfloat16, device=DEV)
    pos = torch.cat([torch.arange(c, c + q) for c, q in zip(b.ctx_lens, b.q_lens)])
    qr_ref = orope.apply_rope(b.q.cpu().unsqueeze(0), b.cos.cpu()[pos].unsqueeze(0),
                              b.sin.cpu()[pos].unsqueeze(0))[0]
    fused = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table,
                                  rope=(b.cos, b.sin, "position"))
    torch.cuda.synchronize()
    assert_close_bf16(fused, oracle_paged(b, qr_ref), "prefill fused rope")
    # decode path with rope by position too
    d = make_batch([10, 500], [1, 1], 32, 8, 128, theta=500000.0)
    dplan = paged.AttentionPlan(d.q_lens, d.seq_lens, num_q_heads=32, num_kv_heads=8, head_dim=128,
                                block_size=16, dtype=torch.bfloat16, device=DEV)
    pos = torch.tensor([10, 500])
    qd = orope.apply_rope(d.q.cpu().unsqueeze(0), d.cos.cpu()[pos].unsqueeze(0), d.sin.cpu()[pos].unsqueeze(0))[0]
    outd = paged.paged_attention(dplan, d.q, d.k_cache, d.v_cache, d.block_table, rope=(d.cos, d.sin, "position"))
    assert_close_bf16(outd, oracle_paged(d, qd), "decode fused rope")


# ------------------------------------------------------------ (d) mixed launch
@pytest.mark.parametrize("split", [256, paged.BALANCED])
def test_mixed_batch_one_launch(split):
    print(f"mixed split={split}", flush=True)
    ctx = [100, 0, 2000, 513, 64, 1000]
    ql = [1, 96, 1, 64, 1, 33]
    b = make_batch(ctx, ql, 32, 8, 128)
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=32, num_kv_heads=8, head_dim=128,
                               block_size=16, dtype=torch.bfloat16, device=DEV, split_tokens=split)
    info = plan.info
    assert info["decode_seqs"] == 3 and info["prefill_seqs"] == 3
    assert (info["decode_segments"] > 0) == (split == paged.BALANCED)
    ref = oracle_paged(b)
    for rep in range(2):   # the second launch finds the split tickets re-armed
        out = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table)
        torch.cuda.synchronize()
        assert_close_bf16(out, ref, f"mixed rep {rep}")


# ------------------------------------------------------------ block sizes
@pytest.mark.parametrize("bs", [1, 3, 12, 24, 48, 100, 1000])
@pytest.mark.parametrize("D,split", [(64, 0), (128, 96), (64, paged.BALANCED), (128, paged.BALANCED)])
def test_any_block_size_mixed(bs, D, split):
    """Block sizes that are not powers of two (the reference takes any
    size): one mixed launch with decodes (split and unsplit), prefill chunks
    with and without context, keys past the prefill kernel's 1024 cached block
    ids at the small sizes, and a prefill whose context starts mid-block."""
    print(f"any block size bs={bs} D={D} split={split}", flush=True)
    ctx = [100, 0, 3500, 513, 7, 1200, 64]
    ql = [1, 96, 1, 64, 1, 40, 1]
    b = make_batch(ctx, ql, 32, 8, D, bs=bs)
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=32, num_kv_heads=8, head_dim=D,
                               block_size=bs, dtype=torch.bfloat16, device=DEV, split_tokens=split)
    assert plan.info["prefill_seqs"] == 3
    ref = oracle_paged(b)
    for rep in range(2):
        out = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table)
        torch.cuda.synchronize()
        assert_close_bf16(out, ref, f"bs {bs} rep {rep}")


@pytest.mark.parametrize("bs", [1, 3, 24, 100])
def test_any_block_size_balanced_decode(bs):
    """Page-balanced decode: segments start on 16-key units, which for these
    block sizes fall inside blocks."""
    print(f"balanced decode bs={bs}", flush=True)
    lens = [1, 9, 16, 47, 130, 511, 2100, 9000]
    b = make_batch([L - 1 for L in lens], [1] * len(lens), 16, 2, 64, bs=bs)
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=16, num_kv_heads=2, head_dim=64,
                               block_size=bs, dtype=torch.bfloat16, device=DEV, split_tokens=paged.BALANCED)
    assert plan.info["decode_segments"] > 0
    ref = oracle_paged(b)
    for rep in range(2):
        out = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table)
        torch.cuda.synchronize()
        assert_close_bf16(out, ref, f"balanced bs {bs} rep {rep}")


@pytest.mark.parametrize("bs", [1, 5, 24])
@pytest.mark.parametrize("kv", [torch.float32, torch.float8_e4m3fn])
def test_any_block_size_fp32(bs, kv):
    print(f"fp32 bs={bs} kv={kv}", flush=True)
    b = make_batch([0, 63, 300, 1000], [70, 1, 9, 1], 8, 2, 64, bs=bs, dtype=torch.float32)
    if kv != torch.float32:
        b.k_cache, b.v_cache = b.k_cache.to(kv), b.v_cache.to(kv)
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=8, num_kv_heads=2, head_dim=64,
                               block_size=bs, dtype=torch.float32, device=DEV)
    out = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table)
    torch.cuda.synchronize()
    d = (out.cpu() - oracle_paged(b)).abs().max().item()
    assert d < 1e-4, d


# ------------------------------------------------------------ other head dims (bf16)
@pytest.mark.parametrize("D", [32, 80, 96, 256])
@pytest.mark.parametrize("kv", [torch.bfloat16, torch.float8_e4m3fn])
def test_bf16_other_head_dims(D, kv):
    """bf16 models with a head dim the MFMA kernels do not take run the
    generic kernel (fp32 arithmetic, q rotated on load with bf16 rounding per
    op): mixed decode + prefill batch, bf16 or fp8 cache, same bar as the
    MFMA paths."""
    print(f"bf16 head dim D={D} kv={kv}", flush=True)
    b = make_batch([0, 63, 300, 1000, 5], [70, 1, 9, 1, 33], 16, 4, D, theta=10000.0)
    if kv != torch.bfloat16:
        b.k_cache, b.v_cache = b.k_cache.to(kv), b.v_cache.to(kv)
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=16, num_kv_heads=4, head_dim=D,
                               block_size=16, dtype=torch.bfloat16, device=DEV)
    out = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table,
                                rope=(b.cos, b.sin, "position"))
    torch.cuda.synchronize()
    pos = torch.cat([torch.arange(c, c + q) for c, q in zip(b.ctx_lens, b.q_lens)])
    q_rot = orope.apply_rope(b.q.cpu().unsqueeze(0), b.cos.cpu()[pos].unsqueeze(0), b.sin.cpu()[pos].unsqueeze(0))[0]
    assert_close_bf16(out, oracle_paged(b, q_rot), f"D={D}")


@pytest.mark.parametrize("D", [48, 96])
def test_bf16_dense_op_other_head_dims(D):
    """reference_attention (dense bias op) for bf16 at other head dims."""
    print(f"bf16 dense D={D}", flush=True)
    g = torch.Generator().manual_seed(D)
    B, Tq, T, Hq, Hkv = 2, 24, 40, 4, 2
    q = torch.randn(B, Tq, Hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, T, Hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, T, Hkv, D, generator=g).to(torch.bfloat16)
    bias = torch.where(torch.rand(B, Tq, T, generator=g) < 0.2, float("-inf"), 0.0).to(torch.bfloat16)
    bias[..., 0] = 0.0
    out = gllm_amd.reference_attention(q.to(DEV), k.to(DEV), v.to(DEV), bias.to(DEV))
    torch.cuda.synchronize()
    ref = oa.reference_attention(q.float(), k.float(), v.float(), bias.float())
    assert_close_bf16(out, ref, f"dense D={D}")


# ------------------------------------------------------------ fp32 path
def test_fp32_paged_parity():
    print("fp32 paged", flush=True)
    b = make_batch([0, 30, 77], [20, 1, 5], 8, 2, 64, dtype=torch.float32)
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=8, num_kv_heads=2, head_dim=64,
                               block_size=16, dtype=torch.float32, device=DEV)
    out = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table)
    torch.cuda.synchronize()
    d = (out.cpu() - oracle_paged(b)).abs().max().item()
    assert d < 1e-4, d


@pytest.mark.parametrize("D,kv", [(64, torch.float32), (128, torch.float32), (50, torch.float32),
                                  (256, torch.float32), (64, torch.bfloat16), (128, torch.float8_e4m3fn)])
def test_fp32_paged_long_contexts(D, kv):
    """fp32 model: keys go 64 per step, so contexts of several steps (with
    ragged last steps and block-boundary lengths), head dims that are not a
    multiple of 4, and bf16 / fp8 caches (widened on load)."""
    print(f"fp32 paged long D={D} kv={kv}", flush=True)
    b = make_batch([0, 63, 64, 65, 300, 1000], [70, 1, 1, 1, 9, 1], 8, 2, D, dtype=torch.float32)
    if kv != torch.float32:
        b.k_cache, b.v_cache = b.k_cache.to(kv), b.v_cache.to(kv)
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=8, num_kv_heads=2, head_dim=D,
                               block_size=16, dtype=torch.float32, device=DEV)
    out = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table)
    torch.cuda.synchronize()
    d = (out.cpu() - oracle_paged(b)).abs().max().item()
    assert d < 1e-4, d


# ------------------------------------------------------------ dense-bias op
@pytest.mark.parametrize("B,Tq,T,Hq,Hkv,D", [(1, 8, 8, 1, 1, 128), (1, 16, 16, 1, 1, 128), (1, 40, 40, 1, 1, 128),
                                             (1, 256, 256, 1, 1, 128), (1, 32, 256, 1, 1, 128),
                                             (1, 32, 256, 2, 1, 128), (8, 32, 256, 1, 1, 128),
                                             (3, 5, 77, 32, 8, 64)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_dense_op_reference_shapes(B, Tq, T, Hq, Hkv, D, dtype):
    """The reference's own op-test shapes (tests/test_attention_op.py:12-34),
    causal-with-offset bias (:56-61), seeded."""
    print(f"dense {B},{Tq},{T},{Hq},{Hkv},{D} {dtype}", flush=True)
    g = torch.Generator().manual_seed(B * 1000 + T + Hq)
    q = torch.randn(B, Tq, Hq, D, generator=g).to(dtype)
    k = torch.randn(B, T, Hkv, D, generator=g).to(dtype)
    v = torch.randn(B, T, Hkv, D, generator=g).to(dtype)
    bias = torch.zeros(B, Tq, T, dtype=dtype)
    bias[:, :, T - Tq:] = torch.full((Tq, Tq), float("-inf")).triu(1).to(dtype)
    ref = oa.reference_attention(q.float(), k.float(), v.float(), bias.float())
    out = gllm_amd.reference_attention(q.to(DEV), k.to(DEV), v.to(DEV), bias.to(DEV))
    torch.cuda.synchronize()
    if dtype == torch.float32:
        assert torch.allclose(out.cpu(), ref, rtol=1e-3, atol=1e-3)   # the reference test's bar
        assert (out.cpu() - ref).abs().max().item() < 1e-4
    else:
        assert_close_bf16(out, ref, "dense bf16")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_dense_op_engine_bias_and_masked_rows(dtype):
    """Left-padded engine bias (llm.py:259-274) and a fully masked row (NaN,
    as torch's softmax)."""
    print(f"dense engine bias {dtype}", flush=True)
    g = torch.Generator().manual_seed(4)
    ctx, ql = [5, 0, 60], [3, 9, 1]
    bt = om.random_block_tables([c + x for c, x in zip(ctx, ql)], 16, 32, g)
    meta = om.build_metadata(ctx, ql, bt, 16, dtype)
    B, Tq, T = meta.bias.shape
    q = torch.randn(B, Tq, 8, 64, generator=g).to(dtype)
    k = torch.randn(B, T, 2, 64, generator=g).to(dtype)
    v = torch.randn(B, T, 2, 64, generator=g).to(dtype)
    bias = meta.bias.clone()
    bias[1, 4, :] = float("-inf")
    ref = oa.reference_attention(q.float(), k.float(), v.float(), bias.float())
    out = gllm_amd.reference_attention(q.to(DEV), k.to(DEV), v.to(DEV), bias.to(DEV)).cpu().float()
    assert torch.isnan(out[1, 4]).all() and torch.isnan(ref[1, 4]).all()
    fin = torch.isfinite(ref)
    d = (out[fin] - ref[fin]).abs()
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    assert d.max().item() < tol


@pytest.mark.parametrize("k", range(12))
def test_dense_op_random_bias(k):
    """reference_attention with arbitrary additive biases (finite values of
    either sign plus scattered -inf, every row keeping a finite entry), seeded
    random shapes, bf16 and fp32."""
    import random
    r = random.Random(500 + k)
    B, Tq = r.randint(1, 4), r.randint(1, 100)
    T = Tq + r.randint(0, 200)
    Hkv = r.choice([1, 2, 4])
    Hq = Hkv * r.choice([1, 2, 4, 8])
    D = r.choice([64, 128])
    dtype = r.choice([torch.float32, torch.bfloat16])
    print(f"dense random {k}: B={B} Tq={Tq} T={T} Hq={Hq} Hkv={Hkv} D={D} {dtype}", flush=True)
    g = torch.Generator().manual_seed(600 + k)
    q = torch.randn(B, Tq, Hq, D, generator=g).to(dtype)
    kk = torch.randn(B, T, Hkv, D, generator=g).to(dtype)
    v = torch.randn(B, T, Hkv, D, generator=g).to(dtype)
    bias = 3.0 * torch.randn(B, Tq, T, generator=g)
    bias[torch.rand(B, Tq, T, generator=g) < 0.3] = float("-inf")
    bias[..., 0] = torch.randn(B, Tq, generator=g)          # a finite entry in every row
    bias = bias.to(dtype)
    ref = oa.reference_attention(q.float(), kk.float(), v.float(), bias.float())
    out = gllm_amd.reference_attention(q.to(DEV), kk.to(DEV), v.to(DEV), bias.to(DEV))
    torch.cuda.synchronize()
    if dtype == torch.float32:
        assert (out.cpu() - ref).abs().max().item() < 1e-4
    else:
        assert_close_bf16(out, ref, "dense random bias")


# ------------------------------------------------------------ call-site drop-in
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_attention_forward_dropin(dtype):
    """gllm_amd.Attention.attention == attention.py:151-178 (oracle) on real
    rows; cache contents bit-exact outside the dummy block."""
    print(f"attention drop-in {dtype}", flush=True)
    g = torch.Generator().manual_seed(21)
    Hq, Hkv, D, bs, nb = 32, 8, 64, 16, 64
    ctx, ql = [0, 33, 100, 7], [12, 1, 1, 20]
    bt = om.random_block_tables([c + x for c, x in zip(ctx, ql)], bs, nb, g, width=16)
    meta = om.build_metadata(ctx, ql, bt, bs, dtype)
    B, Tq = meta.query_slot_mapping.shape
    q = torch.randn(B, Tq, Hq, D, generator=g).to(dtype)
    k = torch.randn(B, Tq, Hkv, D, generator=g).to(dtype)
    v = torch.randn(B, Tq, Hkv, D, generator=g).to(dtype)
    cos_t, sin_t = orope.rope_cache(256, D, 500000.0, dtype)
    cos, sin = cos_t[meta.positions], sin_t[meta.positions]
    kv = torch.randn(2, nb * bs, Hkv, D, generator=g).to(dtype)
    kv_ref = kv.clone()
    ref, _, _ = oa.attention_layer_forward(q, k, v, cos, sin, kv_ref[0], kv_ref[1], meta, sdpa_dtype=torch.float32)

    class Cfg:
        num_attn_heads, num_kv_heads, head_dim, hidden_size = Hq, Hkv, D, Hq * D

    Cfg.dtype = dtype
    w = {f"model.layers.0.self_attn.{n}_proj.weight": torch.zeros(1) for n in "qkvo"}
    att = gllm_amd.Attention(0, Cfg, w)
    gm = gllm_amd.AttentionMetadata(
        query_lens=meta.query_lens.to(DEV), seq_lens=meta.seq_lens.to(DEV), max_seq_len=meta.max_seq_len,
        block_table=meta.block_table.to(DEV), slot_mapping=meta.slot_mapping.to(DEV),
        query_slot_mapping=meta.query_slot_mapping.to(DEV), bias=None, block_size=bs)
    kvd = kv.to(DEV)
    out = att.attention(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV), kvd, gm).cpu()
    assert torch.equal(_bits(kvd)[:, bs:], _bits(kv_ref)[:, bs:])
    for i in range(B):
        if dtype == torch.float32:
            assert (out[i, :ql[i]] - ref[i, :ql[i]]).abs().max().item() < 1e-4
        else:
            assert_close_bf16(out[i, :ql[i]], ref[i, :ql[i]], f"drop-in seq {i}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_attention_layer_forward_real_weights(dtype):
    """gllm_amd.Attention.forward (projections, RoPE, KV write, attention,
    linear_o) == attention.py:122-182 restated by the oracle, on random
    weights; the metadata is the reference's own shape (no block_size: the
    drop-in derives it from the slot mapping)."""
    print(f"attention forward {dtype}", flush=True)
    from dataclasses import dataclass
    import torch.nn.functional as F
    g = torch.Generator().manual_seed(23)
    Hq, Hkv, D, bs, nb = 16, 4, 64, 8, 96
    hidden = Hq * D
    ctx, ql = [0, 40, 9], [17, 1, 1]
    bt = om.random_block_tables([c + x for c, x in zip(ctx, ql)], bs, nb, g, width=12)
    meta = om.build_metadata(ctx, ql, bt, bs, dtype)
    B, Tq = meta.query_slot_mapping.shape
    x = (torch.randn(B, Tq, hidden, generator=g) * 0.5).to(dtype)
    names = {n: f"model.layers.3.self_attn.{n}_proj.weight" for n in "qkvo"}
    w = {names["q"]: torch.randn(Hq * D, hidden, generator=g) / hidden ** 0.5,
         names["k"]: torch.randn(Hkv * D, hidden, generator=g) / hidden ** 0.5,
         names["v"]: torch.randn(Hkv * D, hidden, generator=g) / hidden ** 0.5,
         names["o"]: torch.randn(hidden, Hq * D, generator=g) / hidden ** 0.5}
    cos_t, sin_t = orope.rope_cache(128, D, 500000.0, dtype)
    cos, sin = cos_t[meta.positions], sin_t[meta.positions]
    kv = torch.randn(2, nb * bs, Hkv, D, generator=g).to(dtype)
    kv_ref = kv.clone()
    wq, wk, wv, wo = (w[names[n]].to(dtype) for n in "qkvo")
    # the projections as the drop-in computes them (F.linear on the device), so
    # the RoPE + KV write below can be compared bit for bit
    xd = x.to(DEV)
    q = F.linear(xd, wq.to(DEV)).view(B, Tq, Hq, D).cpu()
    k = F.linear(xd, wk.to(DEV)).view(B, Tq, Hkv, D).cpu()
    v = F.linear(xd, wv.to(DEV)).view(B, Tq, Hkv, D).cpu()
    att_ref, _, _ = oa.attention_layer_forward(q, k, v, cos, sin, kv_ref[0], kv_ref[1], meta,
                                               sdpa_dtype=torch.float32)
    ref = F.linear(att_ref.to(dtype).view(B, Tq, -1).float(), wo.float())

    class Cfg:
        num_attn_heads, num_kv_heads, head_dim, hidden_size = Hq, Hkv, D, hidden

    Cfg.dtype = dtype

    @dataclass
    class RefMeta:            # attention.py:12-26, field for field, no block_size
        query_lens: torch.Tensor
        seq_lens: torch.Tensor
        max_seq_len: int
        block_table: torch.Tensor
        slot_mapping: torch.Tensor
        query_slot_mapping: torch.Tensor
        bias: torch.Tensor

    gm = RefMeta(meta.query_lens.to(DEV), meta.seq_lens.to(DEV), meta.max_seq_len, meta.block_table.to(DEV),
                 meta.slot_mapping.to(DEV), meta.query_slot_mapping.to(DEV), meta.bias.to(DEV))
    att = gllm_amd.Attention(3, Cfg, w)
    kvd = kv.to(DEV)
    out = att.forward(x.to(DEV), cos.to(DEV), sin.to(DEV), kvd, gm).float().cpu()
    assert gm._gllm_plan.block_size == bs
    # K/V written bit-exact outside the dummy block
    assert torch.equal(_bits(kvd)[:, bs:], _bits(kv_ref)[:, bs:])
    tol = 1e-3 if dtype == torch.float32 else 3e-2
    for i in range(B):
        d = (out[i, :ql[i]] - ref[i, :ql[i]]).abs()
        assert d.max().item() < tol, (i, d.max().item())
    # Attention.apply_rope: both tensors bit-identical to attention.py:76-119
    qr, kr = att.apply_rope(q.to(DEV), k.to(DEV), cos.to(DEV), sin.to(DEV))
    assert torch.equal(_bits(qr), _bits(orope.apply_rope(q, cos, sin)))
    assert torch.equal(_bits(kr), _bits(orope.apply_rope(k, cos, sin)))


# ------------------------------------------------------------ errors
def test_errors_are_raised():
    print("errors", flush=True)
    with pytest.raises(NotImplementedError):
        paged.AttentionPlan([1], [10], num_q_heads=8, num_kv_heads=2, head_dim=320, block_size=16,
                            dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        paged.AttentionPlan([5], [3], num_q_heads=8, num_kv_heads=2, head_dim=64, block_size=16,
                            dtype=torch.bfloat16, device=DEV)
    with pytest.raises(AssertionError):
        gllm_amd.reference_attention(torch.zeros(1, 1, 1, 64, device=DEV), torch.zeros(1, 2, 1, 64, device=DEV),
                                     torch.zeros(1, 3, 1, 64, device=DEV), torch.zeros(1, 1, 2, device=DEV))
