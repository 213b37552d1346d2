"""FP8 (e4m3fn) KV cache: the reference's kv_dtype path (gllm/model/layers/
attention.py:160-170 writes k.to(kv_dtype) and reads the gathered window
back with .to(q.dtype)).  Every e4m3 value is a bf16 value, so the kernels'
widened K/V equal the reference's gathered tensors; outputs are checked
against the fp32 oracle reading the same fp8 cache, and the widening itself
exactly (a one-key sequence returns its V row)."""
import pytest
import torch

from gllm_amd import paged
from oracle import attention as oa
from oracle import rope as orope
from tests.gpu_helpers import assert_close_bf16, make_batch, oracle_paged

pytestmark = pytest.mark.gpu
DEV = "cuda"
F8 = torch.float8_e4m3fn


def _fp8(b):
    b.k_cache = b.k_cache.to(F8)
    b.v_cache = b.v_cache.to(F8)
    return b


def _plan(b, **kw):
    return paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=b.num_q_heads, num_kv_heads=b.num_kv_heads,
                               head_dim=b.head_dim, block_size=b.block_size, dtype=b.dtype, device=DEV, **kw)


@pytest.mark.parametrize("Hq,Hkv,D", [(32, 8, 64), (32, 8, 128), (64, 8, 128), (16, 1, 64)])
@pytest.mark.parametrize("split", [0, 96, paged.BALANCED])
def test_fp8_decode_parity(Hq, Hkv, D, split):
    print(f"fp8 decode Hq={Hq} Hkv={Hkv} D={D} split={split}", flush=True)
    b = _fp8(make_batch([0, 15, 16, 300, 1000, 2047], [1] * 6, Hq, Hkv, D))
    out = paged.paged_attention(_plan(b, split_tokens=split), b.q, b.k_cache, b.v_cache, b.block_table)
    torch.cuda.synchronize()
    assert_close_bf16(out, oracle_paged(b), "fp8 decode")


@pytest.mark.parametrize("Hq,Hkv,D", [(32, 8, 128), (32, 8, 64), (8, 1, 64)])
def test_fp8_prefill_parity(Hq, Hkv, D):
    print(f"fp8 prefill Hq={Hq} Hkv={Hkv} D={D}", flush=True)
    b = _fp8(make_batch([0, 37, 300], [130, 77, 45], Hq, Hkv, D))
    out = paged.paged_attention(_plan(b), b.q, b.k_cache, b.v_cache, b.block_table)
    torch.cuda.synchronize()
    assert_close_bf16(out, oracle_paged(b), "fp8 prefill")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("split", [0, paged.BALANCED])
def test_fp8_mixed_parity(D, split):
    """Mixed batch over an fp8 pool: the item plan and the page-balanced
    decode share with prefill items."""
    print(f"fp8 mixed D={D} split={split}", flush=True)
    b = _fp8(make_batch([700, 0, 250, 40, 1500], [1, 90, 1, 33, 1], 32, 8, D))
    plan = _plan(b, split_tokens=split)
    assert plan.info["decode_seqs"] == 3 and plan.info["prefill_seqs"] == 2
    assert (plan.info["decode_segments"] > 0) == (split == paged.BALANCED)
    out = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table)
    torch.cuda.synchronize()
    assert_close_bf16(out, oracle_paged(b), f"fp8 mixed D={D} split={split}")


def test_fp8_cache_under_fp32_model():
    print("fp8 cache, fp32 model", flush=True)
    b = _fp8(make_batch([0, 40, 7], [20, 1, 9], 8, 2, 64, dtype=torch.float32))
    out = paged.paged_attention(_plan(b), b.q, b.k_cache, b.v_cache, b.block_table)
    torch.cuda.synchronize()
    ref = oracle_paged(b)
    d = (out.cpu() - ref).abs()
    assert d.max().item() < 1e-4, d.max().item()


def test_fp8_write_then_attend():
    """New tokens rotated and written into the fp8 cache (rounded like torch's
    cast), then attended with q rotated in the kernel: the reference's
    attention.py:151-178 order on an fp8 pool."""
    print("fp8 write then attend", flush=True)
    b = make_batch([0, 64, 200], [50, 17, 1], 32, 8, 128, theta=500000.0)
    pos = torch.cat([torch.arange(c, c + q) for c, q in zip(b.ctx_lens, b.q_lens)])
    kc, vc = b.k_cache.to(F8), b.v_cache.to(F8)
    kc_ref, vc_ref = kc.cpu().clone(), vc.cpu().clone()
    paged.rope_kv_write(b.k_new, b.v_new, b.cos, b.sin, kc, vc, b.slot_mapping, rope_rows=pos.to(DEV))
    cos, sin = b.cos.cpu()[pos], b.sin.cpu()[pos]
    k_rot = orope.apply_rope(b.k_new.cpu().unsqueeze(0), cos.unsqueeze(0), sin.unsqueeze(0))[0]
    oa.kv_write(kc_ref, vc_ref, b.slot_mapping.cpu(), k_rot, b.v_new.cpu())
    torch.cuda.synchronize()
    assert torch.equal(kc.cpu().view(torch.uint8), kc_ref.view(torch.uint8))
    assert torch.equal(vc.cpu().view(torch.uint8), vc_ref.view(torch.uint8))
    out = paged.paged_attention(_plan(b), b.q, kc, vc, b.block_table, rope=(b.cos, b.sin, "position"))
    q_rot = orope.apply_rope(b.q.cpu().unsqueeze(0), cos.unsqueeze(0), sin.unsqueeze(0))[0]
    ref = oa.paged_attention(q_rot, kc_ref, vc_ref, b.block_table.cpu(), b.ctx_lens, b.q_lens, b.q_row_start,
                             b.block_size)
    torch.cuda.synchronize()
    assert_close_bf16(out, ref, "fp8 write then attend")


@pytest.mark.parametrize("D", [64, 128])
def test_fp8_widening_exact(D):
    """Sequences of one key: the output row is the key's V row, widened from
    fp8 to bf16 by the kernel, so every finite e4m3 code must come back as
    exactly torch's fp8 -> bf16 value (as a value: -0 == +0)."""
    print(f"fp8 widening D={D}", flush=True)
    Hkv = 256 // D
    nseq = 8
    b = make_batch([0] * nseq, [1] * nseq, Hkv, Hkv, D)
    codes = torch.arange(256, dtype=torch.int32)
    codes[(codes & 0x7f) == 0x7f] = 0                      # the two NaN codes
    base = codes.to(torch.uint8).view(F8)
    rows = torch.stack([torch.roll(base, shifts=7 * i) for i in range(nseq)]).reshape(nseq, Hkv, D)  # per-sequence order
    vc = b.v_cache.to(F8)
    kc = b.k_cache.to(F8)
    slots = b.slot_mapping.cpu()
    vcc = vc.cpu()
    vcc[slots] = rows
    vc = vcc.to(DEV)
    out = paged.paged_attention(_plan(b), b.q, kc, vc, b.block_table)
    torch.cuda.synchronize()
    # exact values (the accumulator starts at +0, so code 0x80 = -0.0 comes back as +0.0)
    got, want = out.cpu().float(), rows.to(torch.bfloat16).float()
    assert torch.equal(got, want), (got - want).abs().max().item()


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("split", [0, paged.BALANCED])
@pytest.mark.parametrize("kv8", [False, True])
def test_decode_rope_in_kernel_bit_exact(D, split, kv8):
    """Decode with q rotated in the kernel's prologue returns exactly what the
    same kernel returns for q rotated first by the reference's apply_rope
    (gllm/model/layers/attention.py:105-118, the oracle's restatement): the
    in-register rotation must round like torch's bf16 ops, element for
    element.  An fp8 lane at D = 64 holds one half of each rotate pair and
    loads the other half as well, so that case has its own code."""
    print(f"decode rope fused exact D={D} split={split} kv8={kv8}", flush=True)
    b = make_batch([10, 500, 1999, 63], [1, 1, 1, 1], 32, 8, D, theta=500000.0)
    if kv8:
        b = _fp8(b)
    pos = torch.tensor(b.ctx_lens)
    q_rot = orope.apply_rope(b.q.cpu().unsqueeze(0), b.cos.cpu()[pos].unsqueeze(0), b.sin.cpu()[pos].unsqueeze(0))[0]
    plan = _plan(b, split_tokens=split)
    fused = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table, rope=(b.cos, b.sin, "position"))
    pre = paged.paged_attention(plan, q_rot.to(DEV), b.k_cache, b.v_cache, b.block_table)
    torch.cuda.synchronize()
    assert torch.equal(fused.cpu(), pre.cpu()), (fused.float() - pre.float()).abs().max().item()
    assert_close_bf16(fused, oracle_paged(b, q_rot), "decode fused rope")
