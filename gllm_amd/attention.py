"""Drop-in for ``gllm/model/layers/attention.py``: ``AttentionMetadata`` and
``Attention`` with the hot path (RoPE, KV write, attention) on the HIP kernels.

``Attention.forward`` keeps the reference's signature and semantics
(``attention.py:122-182``): q/k/v projections, rotate-half RoPE, K/V written
to the paged cache through ``query_slot_mapping``, attention of every real
query row over its sequence's keys (mask ``p <= c_i + r``, the 0/-inf pattern
of ``gllm/llm/llm.py:259-274``), then ``linear_o``.  The dense gather through
``slot_mapping`` and the materialised ``bias`` are replaced by kernels that
walk ``block_table``; q is rotated on load inside the attention kernel.
Outputs of padded query rows (``r >= query_lens[i]``) are unspecified, as in
the reference, where they attend to dummy slot 0.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F

from . import paged


@dataclass
class AttentionMetadata:
    """Field-for-field ``attention.py:12-26`` plus the pool's ``block_size``
    (the reference keeps it in ``GeneratorParams``, ``generator_params.py``).
    ``block_size=None`` (and the reference's own metadata object, which has
    no such field) makes :func:`plan_for` derive it from the slot mapping."""

    query_lens: torch.Tensor            # [B] int32
    seq_lens: torch.Tensor              # [B] int32
    max_seq_len: int | torch.Tensor
    block_table: torch.Tensor           # [B, max_num_blocks] int32
    slot_mapping: torch.Tensor          # [B, T] int64 (unused by the kernels)
    query_slot_mapping: torch.Tensor    # [B, T_q] int64
    bias: torch.Tensor | None           # [B, T_q, T] (unused by the kernels)
    block_size: int | None = None


def _block_size(meta, ql: list[int], sl: list[int], hint: int | None = None) -> int:
    """The pool's block size, checked against the metadata itself: the first
    and the last real query row of the longest sequence must sit at
    ``block_table[i][p // bs] * bs + p % bs`` (``llm.py:245-247,277``).  A
    given ``block_size`` that disagrees raises; without one, ``hint`` (the
    size this caller derived before) is taken if it fits, else the unique
    size in 1..1024 that reproduces both slots (one vectorised pass)."""
    i = max(range(len(sl)), key=lambda j: sl[j])
    rows = [0, ql[i] - 1]
    ctx = sl[i] - ql[i]
    slots = [int(x) for x in meta.query_slot_mapping[i, rows].tolist()]
    bt = meta.block_table[i].tolist()
    pos = [ctx + r for r in rows]

    def fits(bs):
        return all(p // bs < len(bt) and bt[p // bs] * bs + p % bs == s for p, s in zip(pos, slots))

    given = getattr(meta, "block_size", None)
    if given is not None:
        if not fits(int(given)):
            raise ValueError(f"block_size {given} does not match the slot mapping (sequence {i}, rows {rows})")
        return int(given)
    if hint is not None and fits(hint):
        return hint
    sizes = np.arange(1, 1025, dtype=np.int64)
    table = np.asarray(bt + [0], dtype=np.int64)
    ok = np.ones_like(sizes, dtype=bool)
    for p, s in zip(pos, slots):
        blk = p // sizes
        inside = blk < len(bt)
        ok &= inside & (table[np.where(inside, blk, len(bt))] * sizes + p % sizes == s)
    cands = sizes[ok].tolist()
    if len(cands) != 1:
        raise ValueError(f"cannot derive the block size from the slot mapping ({len(cands)} candidates); "
                         "set AttentionMetadata.block_size")
    return cands[0]


def plan_for(meta, *, num_q_heads: int, num_kv_heads: int, head_dim: int,
             dtype: torch.dtype, device, block_size_hint: int | None = None) -> paged.AttentionPlan:
    """The batch plan, built once per metadata object (one engine step) and
    reused by every layer.  Reads the lengths back once, like the reference's
    own ``.tolist()`` / ``.item()`` calls in ``llm.py:166,176``.  ``meta`` is
    this module's :class:`AttentionMetadata` or the reference's (no
    ``block_size``: derived from the slot mapping, or ``block_size_hint``
    checked against it)."""
    plan = getattr(meta, "_gllm_plan", None)
    if plan is None:
        ql = meta.query_lens.tolist()
        sl = meta.seq_lens.tolist()
        bs = _block_size(meta, ql, sl, block_size_hint)
        plan = paged.AttentionPlan(ql, sl, num_q_heads=num_q_heads, num_kv_heads=num_kv_heads,
                                   head_dim=head_dim, block_size=bs, dtype=dtype,
                                   device=device, q_seq_stride=meta.query_slot_mapping.shape[1])
        object.__setattr__(meta, "_gllm_plan", plan)
    return plan


class Attention:
    """``attention.py:30-182``.  ``weights`` maps the reference's safetensors
    names (``model.layers.{i}.self_attn.{q,k,v,o}_proj.weight``) to tensors;
    ``model_config`` needs ``dtype, hidden_size, head_dim, num_attn_heads,
    num_kv_heads``."""

    def __init__(self, layer_idx: int, model_config, safetensors):
        self.layer_idx = layer_idx
        self.num_q_heads = model_config.num_attn_heads
        self.num_kv_heads = model_config.num_kv_heads
        self.hidden_size = model_config.hidden_size
        self.head_dim = model_config.head_dim
        assert self.num_q_heads % self.num_kv_heads == 0
        self.num_groups = self.num_q_heads // self.num_kv_heads
        assert self.hidden_size == self.num_q_heads * self.head_dim
        pre = f"model.layers.{layer_idx}.self_attn"
        dt = model_config.dtype
        self.W_q = safetensors[f"{pre}.q_proj.weight"].to(dtype=dt)
        self.W_k = safetensors[f"{pre}.k_proj.weight"].to(dtype=dt)
        self.W_v = safetensors[f"{pre}.v_proj.weight"].to(dtype=dt)
        self.W_o = safetensors[f"{pre}.o_proj.weight"].to(dtype=dt)
        self._block_size = None          # the pool's block size, once derived from a slot mapping

    def apply_rope(self, q: torch.Tensor, k: torch.Tensor, cos_pos: torch.Tensor, sin_pos: torch.Tensor):
        """``attention.py:76-119`` (bit-identical rounding) on the HIP kernel."""
        return paged.rope_rotate(q, cos_pos, sin_pos), paged.rope_rotate(k, cos_pos, sin_pos)

    def forward(self, x: torch.Tensor, cos_pos: torch.Tensor, sin_pos: torch.Tensor,
                kv_cache: torch.Tensor, attention_metadata: AttentionMetadata) -> torch.Tensor:
        B, Tq, hidden = x.shape
        assert hidden == self.hidden_size
        Hq, Hkv, D = self.num_q_heads, self.num_kv_heads, self.head_dim
        q = F.linear(x, self.W_q.to(x.device)).view(B, Tq, Hq, D)
        k = F.linear(x, self.W_k.to(x.device)).view(B, Tq, Hkv, D)
        v = F.linear(x, self.W_v.to(x.device)).view(B, Tq, Hkv, D)
        attn = self.attention(q, k, v, cos_pos, sin_pos, kv_cache, attention_metadata)
        return F.linear(attn.view(B, Tq, -1), self.W_o.to(x.device))

    def attention(self, q, k, v, cos_pos, sin_pos, kv_cache, meta: AttentionMetadata) -> torch.Tensor:
        """The hot path between the projections and ``linear_o``
        (``attention.py:151-178``): returns ``[B, T_q, Hq, D]``."""
        k_cache, v_cache = kv_cache[0], kv_cache[1]
        plan = plan_for(meta, num_q_heads=self.num_q_heads, num_kv_heads=self.num_kv_heads,
                        head_dim=self.head_dim, dtype=q.dtype, device=q.device,
                        block_size_hint=self._block_size)
        self._block_size = plan.block_size
        if paged.fused_kv_write_ok(plan, k_cache.dtype):
            # decode step: the RoPE + KV write inside the attention launch (one
            # launch per layer); the slots are query_slot_mapping's, from the table
            return paged.paged_attention(plan, q, k_cache, v_cache, meta.block_table,
                                         rope=(cos_pos, sin_pos, "row"), kv_new=(k, v))
        paged.rope_kv_write(k, v, cos_pos, sin_pos, k_cache, v_cache, meta.query_slot_mapping,
                            query_lens=meta.query_lens)
        return paged.paged_attention(plan, q, k_cache, v_cache, meta.block_table,
                                     rope=(cos_pos, sin_pos, "row"))
