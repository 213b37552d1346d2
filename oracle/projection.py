"""Restatement of gLLM's q/k/v projections and the fused projection ->
RoPE -> KV-write step (CPU).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows ``gllm/model/layers/linear.py:13-19`` (``F.linear(x, W)`` =
``x @ W^T`` with W stored ``[out, in]``, result in the model dtype) and
``gllm/model/layers/attention.py:139-161`` (q/k/v projections, rotate-half
RoPE on q and k, k/v cast to the cache dtype and stored through the query
slot mapping).
"""
from __future__ import annotations

import torch

from . import rope as _rope


def linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """``linear.py:13-19``: ``x @ w^T`` cast to the model dtype.  The dot
    products are accumulated in fp64 (bf16 x bf16 products are exact there,
    and the sums are within ~2^-40 relative for the test sizes), so each
    output is the correctly rounded model-dtype value of the real dot
    product; torch's own bf16 GEMM accumulates in fp32 and can differ from it
    by one unit in the last place near a rounding boundary."""
    return (x.double() @ w.double().t()).to(x.dtype)


def qkv_rope_kv_write(x, w_q, w_k, w_v, cos_rows, sin_rows, k_cache, v_cache, slots, num_kv_heads, head_dim,
                      real=None):
    """``attention.py:139-161`` for token rows ``x [N, hidden]``.

    ``cos_rows``/``sin_rows [N, D/2]`` are the rows each token rotates with
    (``model.py:195-196``); ``real[N]`` (bool, optional) marks the rows that
    are cached (the reference also writes padded rows, to dummy slot 0;
    callers skip them).  Returns the rotated q ``[N, Hq, D]`` and writes the
    caches in place."""
    n = x.shape[0]
    D = head_dim
    q = linear(x, w_q).view(n, -1, D) if w_q is not None else None
    k = linear(x, w_k).view(n, num_kv_heads, D)
    v = linear(x, w_v).view(n, num_kv_heads, D)
    c, s = cos_rows.unsqueeze(0), sin_rows.unsqueeze(0)
    k = _rope.apply_rope(k.unsqueeze(0), c, s)[0]
    if q is not None:
        q = _rope.apply_rope(q.unsqueeze(0), c, s)[0]
    keep = torch.ones(n, dtype=torch.bool) if real is None else real
    idx = slots[keep]
    k_cache[idx] = k[keep].to(k_cache.dtype)
    v_cache[idx] = v[keep].to(v_cache.dtype)
    return q
