"""Independent fp64 loop implementations used to pin the oracle.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Written from the
mathematics (textbook softmax attention, rotation matrices), not from the
reference's op sequence, with plain Python/numpy loops on tiny inputs.
"""
from __future__ import annotations

import math

import numpy as np


def sdpa_fp64(q, k, v, bias):
    """Textbook ``softmax(q k^T / sqrt(D) + bias) v`` with GQA head
    ``h -> h // G``.  Arrays are numpy; shapes as in ``reference_attention``."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    bias = np.asarray(bias, np.float64)
    B, Tq, Hq, D = q.shape
    T, Hkv = k.shape[1], k.shape[2]
    G = Hq // Hkv
    out = np.zeros((B, Tq, Hq, D))
    for b in range(B):
        for r in range(Tq):
            for h in range(Hq):
                kv = h // G
                s = np.array([sum(q[b, r, h, d] * k[b, t, kv, d] for d in range(D)) / math.sqrt(D)
                              + bias[b, r, t] for t in range(T)])
                mx = s.max()
                if mx == -math.inf:
                    out[b, r, h] = math.nan
                    continue
                e = np.exp(s - mx)
                out[b, r, h] = (e[:, None] * v[b, :, kv, :]).sum(0) / e.sum()
    return out


def rotate_fp64(x, pos, theta):
    """Rotate-half RoPE from its definition: pair (x_j, x_{j+D/2}) is rotated
    by angle ``pos * theta**(-2j/D)`` (a 2x2 rotation matrix)."""
    x = np.asarray(x, np.float64)
    D = x.shape[-1]
    h = D // 2
    out = np.empty_like(x)
    for j in range(h):
        a = pos * theta ** (-2.0 * j / D)
        c, s = math.cos(a), math.sin(a)
        out[..., j] = c * x[..., j] - s * x[..., j + h]
        out[..., j + h] = s * x[..., j] + c * x[..., j + h]
    return out
