"""Device metadata builder against the oracle's restatement of
gllm/llm/llm.py:245-281: query-row slot mapping and positions, bit-exact,
padded and packed layouts."""
import numpy as np
import pytest
import torch

from gllm_amd import paged
from oracle import metadata as om

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(ctx, ql, bs, seed, extra_width=0):
    g = torch.Generator().manual_seed(seed)
    seq = [c + q for c, q in zip(ctx, ql)]
    nb = sum(om.num_required_blocks(L, bs) for L in seq) + 4
    bt = om.random_block_tables(seq, bs, nb, g)
    if extra_width:
        bt = np.concatenate([bt, np.zeros((bt.shape[0], extra_width), dtype=bt.dtype)], axis=1)
    return bt, om.build_metadata(ctx, ql, bt, bs)


CASES = [
    ([0, 5, 31, 16], [7, 1, 1, 33], 16),            # block-boundary crossings, zero context
    ([100, 0, 2047, 3], [1, 64, 1, 1], 16),
    ([0], [1], 16),                                 # single token
    ([15, 16, 17], [1, 1, 1], 16),                  # positions at block edges
    ([250, 9, 40], [3, 70, 12], 32),                # other block size
    ([250, 9, 40], [3, 70, 12], 3),                 # block sizes that are not powers of two
    ([0, 5, 1000], [7, 1, 1], 1),
    ([100, 47, 0], [20, 1, 30], 24),
    ([3000, 1, 99], [1, 300, 2], 100),
    ([1000 + 7 * i for i in range(260)], [1] * 256 + [512] * 4, 16),   # config (d)-like batch
]


@pytest.mark.parametrize("k", range(len(CASES)))
def test_metadata_padded_matches_oracle(k):
    ctx, ql, bs = CASES[k]
    bt, meta = _case(ctx, ql, bs, seed=k)
    B, Tq = len(ql), max(ql)
    btd = torch.from_numpy(bt).to(DEV)
    sl = torch.tensor([c + q for c, q in zip(ctx, ql)], dtype=torch.int32, device=DEV)
    qd = torch.tensor(ql, dtype=torch.int32, device=DEV)
    slots, pos, cu = paged.build_metadata(btd, sl, qd, bs, q_seq_stride=Tq)
    torch.cuda.synchronize()
    assert cu is None
    assert torch.equal(slots.cpu().view(B, Tq), meta.query_slot_mapping)
    assert torch.equal(pos.cpu().view(B, Tq), meta.positions)


@pytest.mark.parametrize("k", range(len(CASES)))
def test_metadata_packed_matches_oracle(k):
    ctx, ql, bs = CASES[k]
    bt, meta = _case(ctx, ql, bs, seed=100 + k, extra_width=3)
    btd = torch.from_numpy(bt).to(DEV)
    sl = torch.tensor([c + q for c, q in zip(ctx, ql)], dtype=torch.int32, device=DEV)
    qd = torch.tensor(ql, dtype=torch.int32, device=DEV)
    slots, pos, cu = paged.build_metadata(btd, sl, qd, bs, num_rows=sum(ql))
    torch.cuda.synchronize()
    ref_slots = torch.cat([meta.query_slot_mapping[i, :q] for i, q in enumerate(ql)])
    ref_pos = torch.cat([meta.positions[i, :q] for i, q in enumerate(ql)])
    assert torch.equal(slots.cpu(), ref_slots)
    assert torch.equal(pos.cpu(), ref_pos)
    assert cu.cpu().tolist() == [0] + np.cumsum(ql).tolist()


def test_metadata_padded_positions_clamped():
    # decode rows padded to a 512-row chunk: c_i + T_q - 1 passes max(seq_len),
    # the kernel clamps padded rows to seq_len - 1 like the oracle
    ctx, ql, bs = [8000, 100, 3000, 0], [1, 512, 1, 3], 16
    bt, meta = _case(ctx, ql, bs, seed=9)
    B, Tq = len(ql), max(ql)
    sl = torch.tensor([c + q for c, q in zip(ctx, ql)], dtype=torch.int32, device=DEV)
    qd = torch.tensor(ql, dtype=torch.int32, device=DEV)
    slots, pos, _ = paged.build_metadata(torch.from_numpy(bt).to(DEV), sl, qd, bs, q_seq_stride=Tq)
    torch.cuda.synchronize()
    p = pos.cpu().view(B, Tq)
    assert torch.equal(p, meta.positions)
    assert int(p.max()) == max(c + q for c, q in zip(ctx, ql)) - 1
    assert p[0].tolist() == [8000] * Tq and p[3].tolist() == [0, 1, 2] + [2] * (Tq - 3)


def test_metadata_never_reads_past_table():
    # a sequence whose length needs more blocks than the table holds: the
    # missing columns give slot 0 instead of reading beyond the row
    bt = torch.tensor([[3, 4], [5, 6]], dtype=torch.int32, device=DEV)
    sl = torch.tensor([40, 20], dtype=torch.int32, device=DEV)     # seq 0 needs 3 blocks of 16
    qd = torch.tensor([40, 4], dtype=torch.int32, device=DEV)
    slots, pos, _ = paged.build_metadata(bt, sl, qd, 16, num_rows=44)
    torch.cuda.synchronize()
    s = slots.cpu().tolist()
    assert s[:16] == [3 * 16 + j for j in range(16)] and s[16:32] == [4 * 16 + j for j in range(16)]
    assert s[32:40] == [0] * 8
    assert s[40:] == [6 * 16 + j for j in range(0, 4)]   # seq 1: positions 16..19 -> block 6
    assert pos.cpu().tolist()[40:] == [16, 17, 18, 19]
