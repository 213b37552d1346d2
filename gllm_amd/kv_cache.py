"""Drop-in for ``gllm/model/kv_cache/paged_kv_cache.py``: the paged pool the
kernels read and write.

Layout (``paged_kv_cache.py:31-44``): ``[2 (K/V), L, NB, block_size, Hkv, D]``
with the per-layer view ``[2, NB * block_size, Hkv, D]``; slot
``block_id * block_size + offset``.  Block 0 is the reserved dummy block.  Block
allocation (``reserve_blocks`` / ``release_blocks``, ``paged_kv_cache.py:
81-110``) stays with the reference's own host allocator: the kernels only
read the block table it fills.
"""
from __future__ import annotations

import torch


class PagedKVCache:
    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, block_size: int,
                 max_batch_size: int, max_seq_len: int, kv_dtype: torch.dtype, device):
        self.block_size = block_size
        nb = self.num_required_blocks(max_batch_size * max_seq_len)
        self.num_blocks = nb
        self.physical_kv_cache = torch.zeros((2, num_layers, nb, block_size, num_kv_heads, head_dim),
                                             dtype=kv_dtype, device=device)
        self.flattened_kv_cache = self.physical_kv_cache.view(2, num_layers, -1, num_kv_heads, head_dim)

    def get_layer_kv_cache(self, layer: int) -> torch.Tensor:
        """``[2, NB * block_size, Hkv, D]`` view of one layer."""
        return self.flattened_kv_cache[:, layer]

    def num_required_blocks(self, num_tokens: int) -> int:
        return 1 + (num_tokens - 1) // self.block_size
