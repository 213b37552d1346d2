"""Restatement of gLLM's batch metadata builder and block allocator (CPU).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows:
* ``gllm/llm/llm.py:233-293``   — slot mapping, left-padded slot mapping,
  0/-inf bias, query slot mapping, positions.
* ``gllm/model/kv_cache/paged_kv_cache.py:46-110`` — free list with block 0
  reserved, LIFO ``pop()``, ref-counted release into ``cached_blocks``.
* ``gllm/model/kv_cache/paged_kv_cache.py:65-66`` — ``num_required_blocks``.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch


def num_required_blocks(num_tokens: int, block_size: int) -> int:
    """``paged_kv_cache.py:65-66``: ``1 + (n - 1) // block_size``."""
    return 1 + (num_tokens - 1) // block_size


class BlockAllocator:
    """Host free-list semantics of ``paged_kv_cache.py:46-50,81-110``.

    Block 0 is a reserved dummy; ids are handed out from the end of the free
    list (highest id first).  Released blocks move to ``cached``; once the free
    list is empty the reference calls ``dict.pop()`` without a key, which
    raises ``TypeError`` whatever ``cached`` holds (``paged_kv_cache.py:55,90``).
    """

    def __init__(self, num_blocks: int):
        self.free = list(range(1, num_blocks))
        self.active: dict[int, int] = {}
        self.cached: dict[int, int] = {}

    def reserve(self, n: int) -> list[int]:
        out = []
        for _ in range(n):
            if self.free:
                bid = self.free.pop()
            else:
                bid = self.cached.pop()  # TypeError, as in the reference
            out.append(bid)
            self.active[bid] = self.active.get(bid, 0) + 1
        return out

    def release(self, ids: list[int]) -> None:
        for bid in ids:
            self.active[bid] -= 1
            if self.active[bid] == 0:
                self.active.pop(bid)
                self.cached[bid] = 0


@dataclass
class Metadata:
    """Field-for-field ``AttentionMetadata`` (``attention.py:12-26``) plus the
    positions ``llm.py:281`` hands to ``Model.forward``."""

    query_lens: torch.Tensor          # [B] int32
    seq_lens: torch.Tensor            # [B] int32
    max_seq_len: torch.Tensor         # 0-d int32 (seq_lens.max())
    block_table: torch.Tensor         # [B, max_num_blocks] int32
    slot_mapping: torch.Tensor        # [B, T] int64 (left-padded)
    query_slot_mapping: torch.Tensor  # [B, T_q] int64
    bias: torch.Tensor                # [B, T_q, T] model dtype, 0 / -inf
    positions: torch.Tensor           # [B, T_q] int64 (padded rows: L_i - 1)


def build_metadata(
    context_lens: list[int],
    query_lens: list[int],
    block_table: np.ndarray,
    block_size: int,
    dtype: torch.dtype = torch.float32,
) -> Metadata:
    """Restates ``llm.py:233-293`` for one batch.

    ``block_table`` is the full ``[B, W]`` int32 table (rows past a sequence's
    own blocks hold 0, as ``llm.py:217`` leaves them).  The row slice to
    ``max_num_blocks`` follows ``llm.py:240-241``.
    """
    B = len(query_lens)
    q = torch.tensor(query_lens, dtype=torch.int32)
    ctx = torch.tensor(context_lens, dtype=torch.int32)
    seq = ctx + q
    nblk = [num_required_blocks(int(s), block_size) for s in seq]
    max_q = int(q.max())
    max_ctx = int(ctx.max())
    max_nb = max(nblk)
    bt = torch.from_numpy(np.ascontiguousarray(block_table[:B, :max_nb])).to(torch.int32)

    # llm.py:245-247 — slot = block_size * block_id + offset, int64.
    offsets = torch.arange(block_size, dtype=torch.int64)
    slots = (block_size * bt.unsqueeze(2) + offsets).view(B, -1)

    T = max_ctx + max_q
    bias = torch.zeros((B, max_q, T), dtype=dtype)
    padded = torch.zeros((B, T), dtype=torch.int64)
    # llm.py:264-268 — context left-padded to max_ctx; pad slots stay 0.
    for i in range(B):
        pad = max_ctx - int(ctx[i])
        L = int(seq[i])
        padded[i, pad:pad + L] = slots[i, :L]
        bias[i, :, :pad] = float("-inf")
    # llm.py:272-274 — causal block over the query columns.
    qb = bias[:, :, max_ctx:]
    qb.fill_(float("-inf"))
    qb.triu_(diagonal=1)
    # llm.py:277, 281.  llm.py:281 gives padded rows (r >= q_i) the position
    # c_i + r too; in a mixed batch that can pass the RoPE table's last row
    # (model.py:195 then raises IndexError).  Padded rows are clamped to the
    # sequence's last position L_i - 1 here, as the product does; real rows
    # keep c_i + r exactly.
    qsm = padded[:, -max_q:].contiguous()
    positions = ctx.to(torch.int64).unsqueeze(1) + torch.arange(max_q, dtype=torch.int64)
    real = torch.arange(max_q).unsqueeze(0) < q.unsqueeze(1)
    positions = torch.where(real, positions, (seq.to(torch.int64) - 1).clamp(min=0).unsqueeze(1))
    return Metadata(
        query_lens=q, seq_lens=seq.to(torch.int32), max_seq_len=seq.max().to(torch.int32),
        block_table=bt, slot_mapping=padded, query_slot_mapping=qsm, bias=bias,
        positions=positions,
    )


def slot_of(block_table_row: np.ndarray, p: int, block_size: int) -> int:
    """Closed form of ``llm.py:245-247`` for one key position."""
    return int(block_table_row[p // block_size]) * block_size + p % block_size


def random_block_tables(
    seq_lens: list[int], block_size: int, num_blocks: int, gen: torch.Generator,
    width: int | None = None,
) -> np.ndarray:
    """Distinct block ids for every sequence, drawn as slices of one
    ``randperm`` of ``[1, num_blocks)`` (block 0 stays the reserved dummy,
    ``paged_kv_cache.py:48-50``)."""
    need = [num_required_blocks(L, block_size) for L in seq_lens]
    if sum(need) > num_blocks - 1:
        raise ValueError("pool too small for the requested sequences")
    W = width if width is not None else max(need)
    perm = torch.randperm(num_blocks - 1, generator=gen).numpy().astype(np.int32) + 1
    bt = np.zeros((len(seq_lens), W), dtype=np.int32)
    o = 0
    for i, n in enumerate(need):
        bt[i, :n] = perm[o:o + n]
        o += n
    return bt
