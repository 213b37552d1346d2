"""Restatement of gLLM's RoPE table and rotation (CPU).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows ``gllm/model/model.py:117-128`` (table) and
``gllm/model/layers/attention.py:76-119`` (rotate-half rotation, each op
rounded to the model dtype).
"""
from __future__ import annotations

import torch


def rope_cache(max_seq_len: int, head_dim: int, theta: float, dtype: torch.dtype):
    """``model.py:117-128``: fp32 ``theta**(-2m/D)``, fp32 ``p*theta_m``,
    fp32 cos/sin, then a cast to the model dtype.  Returns (cos, sin), each
    ``[max_seq_len, head_dim // 2]``."""
    p = torch.arange(max_seq_len)
    m = torch.arange(head_dim // 2)
    inv = theta ** (-2 * m / head_dim)          # int64 / int -> float32
    ang = p.unsqueeze(1) * inv                  # int64 * float32 -> float32
    return torch.cos(ang).to(dtype), torch.sin(ang).to(dtype)


def apply_rope(x: torch.Tensor, cos_pos: torch.Tensor, sin_pos: torch.Tensor) -> torch.Tensor:
    """``attention.py:91-118`` for one tensor ``x [B, T_q, H, D]`` with
    ``cos_pos/sin_pos [B, T_q, D/2]`` in the same dtype.

    The first half of the head dim pairs with the second half (not
    interleaved).  Each multiply and the add/sub are separate torch ops, so
    every intermediate is rounded to ``x.dtype`` exactly as the reference
    rounds it.
    """
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h], x[..., h:]
    c = cos_pos.unsqueeze(2)
    s = sin_pos.unsqueeze(2)
    a = x1 * c
    b = x2 * s
    lo = a - b
    e = x1 * s
    f = x2 * c
    hi = e + f
    return torch.cat([lo, hi], dim=-1)
