"""Host-side logic of the drop-in call site (no GPU): the block size the
plan uses is derived from, or checked against, the batch's slot mapping
(gllm/llm/llm.py:245-247,277), since the reference's AttentionMetadata
(attention.py:12-26) carries no block_size."""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from gllm_amd.attention import _block_size
from oracle import metadata as om


@pytest.mark.parametrize("bs", [1, 3, 8, 16, 24, 64])
def test_block_size_derived_from_slot_mapping(bs):
    g = torch.Generator().manual_seed(bs)
    ctx, ql = [5, 70, 0, 33], [1, 1, 12, 3]
    bt = om.random_block_tables([c + q for c, q in zip(ctx, ql)], bs, 400, g)
    m = om.build_metadata(ctx, ql, bt, bs)
    meta = SimpleNamespace(query_slot_mapping=m.query_slot_mapping, block_table=m.block_table)
    assert _block_size(meta, ql, [c + q for c, q in zip(ctx, ql)]) == bs
    meta.block_size = bs
    assert _block_size(meta, ql, [c + q for c, q in zip(ctx, ql)]) == bs


def test_wrong_block_size_raises():
    g = torch.Generator().manual_seed(3)
    ctx, ql = [40, 3], [1, 9]
    bt = om.random_block_tables([c + q for c, q in zip(ctx, ql)], 8, 200, g)
    m = om.build_metadata(ctx, ql, bt, 8)
    meta = SimpleNamespace(query_slot_mapping=m.query_slot_mapping, block_table=m.block_table, block_size=16)
    with pytest.raises(ValueError, match="does not match"):
        _block_size(meta, ql, [c + q for c, q in zip(ctx, ql)])


def test_block_size_hint_and_vectorised_search():
    """The search over 1..1024 agrees with a per-size brute force, an
    ambiguous slot map takes a hint that fits, a hint that does not fit is
    ignored, and one derivation for a 256-sequence batch costs well under a
    millisecond of host time per call (the plan is built once per step)."""
    import time
    g = torch.Generator().manual_seed(11)
    ctx = [int(x) for x in torch.randint(100, 3000, (256,), generator=g)]
    ql = [1] * 256
    bt = om.random_block_tables([c + q for c, q in zip(ctx, ql)], 16, 60000, g)
    m = om.build_metadata(ctx, ql, bt, 16)
    meta = SimpleNamespace(query_slot_mapping=m.query_slot_mapping, block_table=m.block_table)
    sl = [c + q for c, q in zip(ctx, ql)]
    t0 = time.perf_counter()
    for _ in range(20):
        assert _block_size(meta, ql, sl) == 16
    assert (time.perf_counter() - t0) / 20 < 5e-3
    assert _block_size(meta, ql, sl, hint=16) == 16
    assert _block_size(meta, ql, sl, hint=8) == 16         # a hint that does not fit is not taken
    # a table starting at block 0 (slot == position for every size above the
    # positions): sizes 3..1024 all reproduce the slots -> ambiguous
    meta1 = SimpleNamespace(query_slot_mapping=torch.tensor([[1, 2]]),
                            block_table=torch.tensor([[0, 5, 0]], dtype=torch.int32))
    with pytest.raises(ValueError, match="candidates"):
        _block_size(meta1, [2], [3])
    assert _block_size(meta1, [2], [3], hint=8) == 8
