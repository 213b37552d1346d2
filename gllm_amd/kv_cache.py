"""Drop-in for ``gllm/model/kv_cache/paged_kv_cache.py``: the paged pool the
kernels read and write.

Layout (``paged_kv_cache.py:31-44``): ``[2 (K/V), L, NB, block_size, Hkv, D]``
with the per-layer view ``[2, NB * block_size, Hkv, D]``; slot
``block_id * block_size + offset``.  Block 0 is the reserved dummy block.  The
allocator keeps the reference's host semantics (LIFO free list, ref-counted
release into a cache that is never handed out again: once the free list is
empty ``reserve_blocks`` raises ``TypeError``, as ``dict.pop()`` does there).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class GPUBlock:
    id: int
    ref_count: int = 0


class PagedKVCache:
    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, block_size: int,
                 max_batch_size: int, max_seq_len: int, kv_dtype: torch.dtype, device):
        self.block_size = block_size
        nb = self.num_required_blocks(max_batch_size * max_seq_len)
        self.num_blocks = nb
        self.physical_kv_cache = torch.zeros((2, num_layers, nb, block_size, num_kv_heads, head_dim),
                                             dtype=kv_dtype, device=device)
        self.flattened_kv_cache = self.physical_kv_cache.view(2, num_layers, -1, num_kv_heads, head_dim)
        self.free_blocks = [GPUBlock(i) for i in range(1, nb)]
        self.active_blocks: dict[int, GPUBlock] = {}
        self.cached_blocks: dict[int, GPUBlock] = {}

    def get_layer_kv_cache(self, layer: int) -> torch.Tensor:
        """``[2, NB * block_size, Hkv, D]`` view of one layer."""
        return self.flattened_kv_cache[:, layer]

    def num_required_blocks(self, num_tokens: int) -> int:
        return 1 + (num_tokens - 1) // self.block_size

    def reserve_blocks(self, num_blocks: int) -> list[int]:
        ids = []
        for _ in range(num_blocks):
            if self.free_blocks:
                block = self.free_blocks.pop()
            else:
                raise TypeError("KV pool exhausted: no free blocks left (cached blocks are not recycled)")
            ids.append(block.id)
            self.active_blocks[block.id] = block
            block.ref_count += 1
        return ids

    def release_blocks(self, block_ids: list[int]) -> None:
        for bid in block_ids:
            block = self.active_blocks[bid]
            block.ref_count -= 1
            if block.ref_count == 0:
                self.active_blocks.pop(bid)
                self.cached_blocks[bid] = block
