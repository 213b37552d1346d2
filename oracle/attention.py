"""Restatement of gLLM's attention op and call site (CPU, torch).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows:
* ``gllm/ops/attention/reference_attention.py:5-51`` — GQA-expanded dense
  SDPA with an additive bias.
* ``gllm/model/layers/attention.py:151-178`` — RoPE, KV write through
  ``query_slot_mapping``, KV gather through ``slot_mapping`` (with the
  kv_dtype round trip), then the op.
"""
from __future__ import annotations

import math

import torch

from .metadata import Metadata
from .rope import apply_rope


def reference_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                        bias: torch.Tensor) -> torch.Tensor:
    """``reference_attention.py:5-51``.

    q ``[B,T_q,Hq,D]``, k/v ``[B,T,Hkv,D]``, bias ``[B,T_q,T]`` ->
    ``[B,T_q,Hq,D]``.  Query head ``h`` reads kv head ``h // G``
    (``:19-30``); scores are ``(q @ k^T) / sqrt(D)`` (``:40``) plus the bias
    (``:42``), softmax over keys (``:45``), times V (``:48``).  A row whose
    bias is all ``-inf`` comes out NaN, as torch's softmax makes it.
    """
    assert k.shape == v.shape
    B, Tq, Hq, D = q.shape
    Hkv = k.shape[2]
    G = Hq // Hkv
    if G > 1:
        k = torch.repeat_interleave(k, G, dim=2)
        v = torch.repeat_interleave(v, G, dim=2)
    qh = q.transpose(1, 2)
    kh = k.transpose(1, 2)
    vh = v.transpose(1, 2)
    s = torch.matmul(qh, kh.transpose(-2, -1)) / D ** 0.5
    s = s + bias.unsqueeze(1)
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, vh).transpose(1, 2).contiguous()


def kv_write(k_cache: torch.Tensor, v_cache: torch.Tensor, query_slot_mapping: torch.Tensor,
             k: torch.Tensor, v: torch.Tensor) -> None:
    """``attention.py:156-161``: every (padded) query row writes its slot;
    padded rows write slot 0 of the reserved dummy block."""
    Hkv, D = k.shape[-2], k.shape[-1]
    idx = query_slot_mapping.reshape(-1)
    k_cache[idx] = k.reshape(-1, Hkv, D).to(k_cache.dtype)
    v_cache[idx] = v.reshape(-1, Hkv, D).to(v_cache.dtype)


def kv_gather(cache: torch.Tensor, slot_mapping: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """``attention.py:165-170``: dense ``[B, T, Hkv, D]`` window cast back to
    the model dtype."""
    B = slot_mapping.shape[0]
    Hkv, D = cache.shape[-2], cache.shape[-1]
    return cache[slot_mapping.reshape(-1)].view(B, -1, Hkv, D).to(dtype)


def attention_layer_forward(q, k, v, cos_pos, sin_pos, k_cache, v_cache, meta: Metadata,
                            sdpa_dtype: torch.dtype | None = None):
    """``attention.py:151-178`` (between the projections and ``linear_o``).

    q ``[B,T_q,Hq,D]``, k/v ``[B,T_q,Hkv,D]`` (pre-RoPE), cos/sin
    ``[B,T_q,D/2]``.  Mutates the caches like the reference.  The dense op runs
    in ``sdpa_dtype`` (default: the model dtype, as in the reference); pass
    ``torch.float32`` to get "the reference fp32 result" for bf16 inputs.
    """
    qr = apply_rope(q, cos_pos, sin_pos)
    kr = apply_rope(k, cos_pos, sin_pos)
    kv_write(k_cache, v_cache, meta.query_slot_mapping, kr, v)
    kg = kv_gather(k_cache, meta.slot_mapping, q.dtype)
    vg = kv_gather(v_cache, meta.slot_mapping, q.dtype)
    dt = sdpa_dtype or q.dtype
    out = reference_attention(qr.to(dt), kg.to(dt), vg.to(dt), meta.bias.to(dt))
    return out, qr, kr


def paged_attention(q_rows: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                    block_table: torch.Tensor, context_lens: list[int], query_lens: list[int],
                    q_row_start: list[int], block_size: int, scale: float | None = None,
                    dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Per-sequence attention straight from the paged cache.

    This is the reference's path on every real query row: key position ``p``
    of sequence ``i`` lives at ``slot = bt[i, p // bs] * bs + p % bs``
    (``llm.py:245-247``) and is visible to query row ``r < q_i`` iff
    ``p <= c_i + r`` (the 0/-inf pattern ``llm.py:264-274`` builds, on real
    rows).  ``q_rows`` is ``[rows, Hq, D]`` with sequence ``i``'s rows at
    ``q_row_start[i] .. + q_i``.  Returns ``[rows, Hq, D]`` in ``dtype``;
    rows not owned by any sequence are left zero.  Cached K/V are read as
    the reference's gather reads them, cast to the model dtype (``q_rows``'
    dtype, ``attention.py:169-170``), and only then widened to ``dtype``.
    """
    Hq, D = q_rows.shape[-2], q_rows.shape[-1]
    Hkv = k_cache.shape[-2]
    G = Hq // Hkv
    sc = (1.0 / math.sqrt(D)) if scale is None else scale
    out = torch.zeros(q_rows.shape, dtype=dtype)
    for i, (c, qn, r0) in enumerate(zip(context_lens, query_lens, q_row_start)):
        L = c + qn
        if qn == 0:
            continue
        p = torch.arange(L)
        slots = block_table[i, p // block_size].to(torch.int64) * block_size + p % block_size
        kk = k_cache[slots].to(q_rows.dtype).to(dtype)   # [L, Hkv, D]; the gather's cast, then fp32
        vv = v_cache[slots].to(q_rows.dtype).to(dtype)
        qq = q_rows[r0:r0 + qn].to(dtype)           # [qn, Hq, D]
        kk = torch.repeat_interleave(kk, G, dim=1)  # head h -> kv head h // G
        vv = torch.repeat_interleave(vv, G, dim=1)
        s = torch.einsum("rhd,phd->hrp", qq, kk) * sc
        vis = p.unsqueeze(0) <= (c + torch.arange(qn)).unsqueeze(1)   # [qn, L]
        s = s.masked_fill(~vis.unsqueeze(0), float("-inf"))
        pr = torch.softmax(s, dim=-1)
        out[r0:r0 + qn] = torch.einsum("hrp,phd->rhd", pr, vv)
    return out


def lse_merge(ms, ls, accs):
    """Combines split-context partials ``(m_s, l_s, acc_s)`` — running max,
    sum of ``exp(s - m_s)`` and unnormalised ``sum exp(s - m_s) v`` — into the
    one-shot softmax output (natural-exp convention)."""
    M = torch.stack(ms).max(dim=0).values
    w = [torch.exp(m - M) for m in ms]
    L = sum(wi * li for wi, li in zip(w, ls))
    O = sum(wi.unsqueeze(-1) * a for wi, a in zip(w, accs))
    return O / L.unsqueeze(-1)
