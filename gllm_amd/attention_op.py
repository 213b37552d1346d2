"""Drop-in for ``gllm/ops/attention/reference_attention.py`` and
``gllm/ops/attention/flash_attention.py``: the dense-bias attention op on the
HIP kernels (bf16 / fp16 MFMA, or the generic fp32-arithmetic kernel)."""
from __future__ import annotations

import math

import torch

from . import _lib


def reference_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """Same contract as ``reference_attention.py:5-51``: q ``[B,T_q,Hq,D]``,
    k/v ``[B,T,Hkv,D]``, bias ``[B,T_q,T]`` -> new ``[B,T_q,Hq,D]``.  Query
    head h reads kv head h // (Hq / Hkv); scores are scaled by 1/sqrt(D).
    Inputs are not mutated; a fully -inf bias row gives NaN, like torch."""
    assert k.shape == v.shape
    B, Tq, Hq, D = q.shape
    _, T, Hkv, _ = k.shape
    if Hq % Hkv:
        raise ValueError("num_q_heads must be a multiple of num_kv_heads")
    if bias.shape != (B, Tq, T):
        raise ValueError(f"bias must be [B, T_q, T] = {(B, Tq, T)}, got {tuple(bias.shape)}")
    q = q.contiguous()
    if k.stride(-1) != 1 or k.stride(-2) != D:
        k = k.contiguous()
    if v.stride(-1) != 1 or v.stride(-2) != D:
        v = v.contiguous()
    bias = bias.to(q.dtype)
    if bias.stride(-1) != 1:
        bias = bias.contiguous()
    out = torch.empty_like(q)
    lib = _lib.load()
    _lib.check(lib.gllm_attention_dense(
        q.data_ptr(), Hq * D, k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1),
        bias.data_ptr(), bias.stride(0), bias.stride(1), out.data_ptr(), Hq * D, B, Tq, T, Hq, Hkv, D,
        1.0 / math.sqrt(D), _lib.dtype_code(q.dtype), _lib.stream_ptr(q.device)))
    return out


# ``flash_attention`` (flash_attention.py:155-192) has the same contract.
flash_attention = reference_attention
