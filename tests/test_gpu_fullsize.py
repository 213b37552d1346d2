"""GPU parity at the benchmark configurations' full sizes.

Where the CPU oracle would take too long on every row, rows are sampled: a
query row r of sequence i is checked as its own one-row "sequence" with
context c_i + r over the same block-table row, which sees exactly the keys
p <= c_i + r the row sees in the batch.  Size-independent properties cover
the rest: the result must not depend on the decode workgroup shape or the
split length (split-context LSE merge == one-shot softmax).
"""
import pytest
import torch

from gllm_amd import paged, workloads
from oracle import attention as oa
from oracle import rope as orope
from tests.gpu_helpers import assert_close_bf16

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _plan(b, **kw):
    return paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=b.num_q_heads, num_kv_heads=b.num_kv_heads,
                               head_dim=b.head_dim, block_size=b.block_size, dtype=b.dtype, device=DEV, **kw)


def _sample_rows(b, seqs, rows_per_seq, gen):
    """(seq, row) pairs: first, last and random rows of the chosen sequences."""
    out = []
    for i in seqs:
        q = b.q_lens[i]
        rs = {0, q - 1}
        if q > 2:
            rs |= set(torch.randint(0, q, (min(rows_per_seq, q),), generator=gen).tolist())
        out += [(i, r) for r in sorted(rs)]
    return out


def _oracle_rows(b, pairs, q_rows):
    """fp32 oracle for sampled rows; gathers only the touched blocks."""
    bs = b.block_size
    bt = b.block_table.cpu()
    need = sorted({int(x) for i, r in pairs for x in bt[i, :-(-(b.ctx_lens[i] + r + 1) // bs)]})
    remap = {blk: j for j, blk in enumerate(need)}
    idx = torch.tensor(need, dtype=torch.int64, device=b.k_cache.device)
    kc = b.k_cache.view(-1, bs, b.num_kv_heads, b.head_dim)[idx].reshape(-1, b.num_kv_heads, b.head_dim).cpu()
    vc = b.v_cache.view(-1, bs, b.num_kv_heads, b.head_dim)[idx].reshape(-1, b.num_kv_heads, b.head_dim).cpu()
    width = max(-(-(b.ctx_lens[i] + r + 1) // bs) for i, r in pairs)
    sbt = torch.zeros(len(pairs), width, dtype=torch.int32)
    for k, (i, r) in enumerate(pairs):
        n = -(-(b.ctx_lens[i] + r + 1) // bs)
        sbt[k, :n] = torch.tensor([remap[int(x)] for x in bt[i, :n]], dtype=torch.int32)
    qs = torch.stack([q_rows[b.q_row_start[i] + r] for i, r in pairs])
    return oa.paged_attention(qs, kc, vc, sbt, [b.ctx_lens[i] + r for i, r in pairs], [1] * len(pairs),
                              list(range(len(pairs))), bs)


def test_config_b_decode_full():
    print("config b full", flush=True)
    b = workloads.materialize(workloads.config_b(), DEV, values_on_device=True)
    ref = _oracle_rows(b, [(i, 0) for i in range(len(b.q_lens))], b.q.cpu())
    outs = []
    B = paged.BALANCED
    for hw, split in ((0, 0), (1, 0), (2, 0), (4, 0), (8, 0), (2, 256), (8, 128), (0, B), (2, B), (4, B), (1, B)):
        out = paged.paged_attention(_plan(b, heads_per_wg=hw, split_tokens=split), b.q, b.k_cache, b.v_cache,
                                    b.block_table)
        torch.cuda.synchronize()
        assert_close_bf16(out, ref, f"config b hw={hw} split={split}")
        outs.append(out.float().cpu())
    for o in outs[1:]:   # workgroup shape / split invariance: at most 1-2 bf16 ulps apart
        assert (o - outs[0]).abs().max().item() < 2e-2


def test_config_b_decode_full_fp8():
    """Config (b) over an fp8 (e4m3fn) pool: 512 decode workgroups of one kv
    head each, which the kernel regroups by XCD in blocks of 64 (eight full
    blocks here: a mapping that ran an item twice and another never would
    leave rows unwritten); every row against the fp32 oracle on the same fp8
    cache, and the result independent of the workgroup shape."""
    print("config b full fp8", flush=True)
    cb = workloads.config_b()
    cb.kv_dtype = torch.float8_e4m3fn
    b = workloads.materialize(cb, DEV, values_on_device=True)
    assert b.k_cache.dtype == torch.float8_e4m3fn
    ref = _oracle_rows(b, [(i, 0) for i in range(len(b.q_lens))], b.q.cpu())
    outs = []
    for hw, split in ((0, 0), (1, 0), (2, 0), (8, 128), (0, paged.BALANCED)):
        plan = _plan(b, heads_per_wg=hw, split_tokens=split)
        if hw == 0 and split == 0:
            assert plan.info["heads_per_wg"] == 1 and plan.info["work_items"] == 512
        out = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table)
        torch.cuda.synchronize()
        assert_close_bf16(out, ref, f"config b fp8 hw={hw} split={split}")
        outs.append(out.float().cpu())
    for o in outs[1:]:
        assert (o - outs[0]).abs().max().item() < 2e-2


def test_config_c_prefill_full():
    print("config c full", flush=True)
    b = workloads.materialize(workloads.config_c(), DEV, values_on_device=True)
    pos = torch.cat([torch.arange(c, c + q) for c, q in zip(b.ctx_lens, b.q_lens)])
    paged.rope_kv_write(b.k_new, b.v_new, b.cos, b.sin, b.k_cache, b.v_cache, b.slot_mapping, rope_rows=pos.to(DEV))
    out = paged.paged_attention(_plan(b), b.q, b.k_cache, b.v_cache, b.block_table, rope=(b.cos, b.sin, "position"))
    torch.cuda.synchronize()
    g = torch.Generator().manual_seed(9)
    # KV write bit-exact for sampled tokens (oracle rope in bf16 on the CPU)
    toks = torch.randint(0, b.rows, (512,), generator=g)
    cos, sin = b.cos.cpu()[pos[toks]], b.sin.cpu()[pos[toks]]
    kref = orope.apply_rope(b.k_new.cpu()[toks].unsqueeze(0), cos.unsqueeze(0), sin.unsqueeze(0))[0]
    slots = b.slot_mapping.cpu()[toks]
    assert torch.equal(b.k_cache[slots.to(DEV)].cpu().view(torch.int16), kref.view(torch.int16))
    assert torch.equal(b.v_cache[slots.to(DEV)].cpu().view(torch.int16), b.v_new.cpu()[toks].view(torch.int16))
    # attention: sampled rows of every sequence, q rotated as the kernel does
    pairs = _sample_rows(b, range(len(b.q_lens)), 24, g)
    prow = torch.tensor([b.ctx_lens[i] + r for i, r in pairs])
    qrows = torch.stack([b.q.cpu()[b.q_row_start[i] + r] for i, r in pairs])
    qrot = orope.apply_rope(qrows.unsqueeze(0), b.cos.cpu()[prow].unsqueeze(0), b.sin.cpu()[prow].unsqueeze(0))[0]
    qfull = b.q.cpu().clone()
    for k, (i, r) in enumerate(pairs):
        qfull[b.q_row_start[i] + r] = qrot[k]
    ref = _oracle_rows(b, pairs, qfull)
    got = torch.stack([out[b.q_row_start[i] + r].cpu() for i, r in pairs])
    assert_close_bf16(got, ref, "config c sampled rows")


@pytest.mark.parametrize("split", [0, paged.BALANCED])
def test_config_d_mixed_full(split):
    """Config (d) in one launch: the item plan, and the page-balanced decode
    share with prefill items (twice: the split tickets are re-armed)."""
    print(f"config d full split={split}", flush=True)
    b = workloads.materialize(workloads.config_d(), DEV, values_on_device=True)
    plan = _plan(b, split_tokens=split)
    assert plan.info["decode_seqs"] == 256 and plan.info["prefill_seqs"] == 4
    assert (plan.info["decode_segments"] > 0) == (split == paged.BALANCED)
    for _ in range(2 if split else 1):
        out = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table)
    torch.cuda.synchronize()
    g = torch.Generator().manual_seed(10)
    pairs = [(i, 0) for i in torch.randint(0, 256, (48,), generator=g).tolist()]
    pairs += _sample_rows(b, range(256, 260), 24, g)
    ref = _oracle_rows(b, pairs, b.q.cpu())
    got = torch.stack([out[b.q_row_start[i] + r].cpu() for i, r in pairs])
    assert_close_bf16(got, ref, "config d sampled rows")


def test_config_e_long_decode():
    print("config e full", flush=True)
    b = workloads.materialize(workloads.config_e(), DEV, values_on_device=True)
    out = paged.paged_attention(_plan(b), b.q, b.k_cache, b.v_cache, b.block_table)
    assert _plan(b).info["decode_segments"] > 0       # long contexts: page-balanced plan
    out2 = paged.paged_attention(_plan(b, heads_per_wg=8, split_tokens=2048), b.q, b.k_cache, b.v_cache,
                                 b.block_table)
    torch.cuda.synchronize()
    assert (out.float() - out2.float()).abs().max().item() < 2e-2     # split invariance
    g = torch.Generator().manual_seed(11)
    pairs = [(i, 0) for i in torch.randint(0, 128, (12,), generator=g).tolist()]
    ref = _oracle_rows(b, pairs, b.q.cpu())
    got = torch.stack([out[b.q_row_start[i]].cpu() for i, r in pairs])
    assert_close_bf16(got, ref, "config e sampled rows")
