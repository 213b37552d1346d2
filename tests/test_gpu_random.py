"""Seeded random batches through every planner and cache dtype, against the
fp32 oracle (oracle/attention.py::paged_attention, the restatement of
reference_attention.py:5-51 over the paged cache with the mask of
llm.py:259-274).

Each case draws head counts, head dim, block size, cache dtype and a batch
that mixes decode rows (one query row, contexts from 0 up to a few thousand
keys, block-size boundaries included) with prefill rows (chunks on top of
contexts), so the planners see shapes the hand-written tests do not: ragged
row blocks, every G in 1 .. 8 (G = 3, 5, 6, 7 give decode tiles whose
rows do not divide 16), single-key sequences, decode-only batches under the
split and page-balanced planners, and RoPE applied on load.
"""
import os
import random

import pytest
import torch

from gllm_amd import paged
from oracle import rope as orope
from tests.gpu_helpers import assert_close_bf16, make_batch, oracle_paged

pytestmark = pytest.mark.gpu
DEV = "cuda"
F8 = torch.float8_e4m3fn
# GLLM_RANDOM_CASES=n draws n seeded cases instead of the default 96
N_CASES = int(os.environ.get("GLLM_RANDOM_CASES", "96"))


def _case(k):
    r = random.Random(1000 + k)
    Hkv = r.choice([1, 2, 4, 8])
    G = r.choice([1, 2, 3, 4, 5, 6, 7, 8])   # 3, 5, 6, 7: R = q_len * G does not divide 16
    D = r.choice([64, 128])
    bs = r.choice([8, 16, 32])
    kv8 = r.random() < 0.3
    decode_only = r.random() < 0.4
    nseq = r.randint(1, 12)
    ctx, ql = [], []
    for _ in range(nseq):
        if decode_only or r.random() < 0.6:
            c = r.choice([0, 1, bs - 1, bs, bs + 1, r.randint(0, 3000)])
            ctx.append(c)
            ql.append(1)
        else:
            ctx.append(r.choice([0, r.randint(0, 700)]))
            ql.append(r.randint(2, 200))
    # a decode row whose query heads do not fit one 16-row MFMA tile goes to
    # the prefill path; either path must agree with the oracle
    rope = r.random() < 0.5
    split = r.choice([0, 0, 32, 96, 256, paged.BALANCED]) if decode_only else 0
    hw = r.choice([0, 0, 1, 2, 4, 8])
    if not decode_only and r.random() < 0.35:
        split = paged.BALANCED   # mixed page-balanced plan (prefill items after the decode share)
    return dict(Hq=Hkv * G, Hkv=Hkv, D=D, bs=bs, kv8=kv8, ctx=ctx, ql=ql, rope=rope, split=split, hw=hw)


@pytest.mark.parametrize("k", range(N_CASES))
def test_random_batch(k):
    c = _case(k)
    print(f"random case {k}: {c}", flush=True)
    b = make_batch(c["ctx"], c["ql"], c["Hq"], c["Hkv"], c["D"], bs=c["bs"], theta=500000.0 if c["rope"] else None)
    if c["kv8"]:
        b.k_cache, b.v_cache = b.k_cache.to(F8), b.v_cache.to(F8)
    split = c["split"]
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=c["Hq"], num_kv_heads=c["Hkv"], head_dim=c["D"],
                               block_size=c["bs"], dtype=torch.bfloat16, device=DEV, split_tokens=split,
                               heads_per_wg=c["hw"])
    q_ref = None
    kw = {}
    if c["rope"]:
        pos = torch.cat([torch.arange(cc, cc + q) for cc, q in zip(b.ctx_lens, b.q_lens)])
        q_ref = orope.apply_rope(b.q.cpu().unsqueeze(0), b.cos.cpu()[pos].unsqueeze(0), b.sin.cpu()[pos].unsqueeze(0))[0]
        kw["rope"] = (b.cos, b.sin, "position")
    out = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table, **kw)
    torch.cuda.synchronize()
    assert_close_bf16(out, oracle_paged(b, q_ref), f"random case {k}")
