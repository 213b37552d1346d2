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
