"""Restatement of gLLM's engine path for a Llama-shaped model (CPU, fp32).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Used for benchmark config (a): a random-init Llama-3.2-1B-shaped model run
through the reference's batching path, recording per-layer attention outputs
and the greedy tokens.  Follows:

* ``gllm/model/model.py:117-128,185-239`` — RoPE table, cos/sin gather by
  positions, layer loop, final norm, tied-embedding logits.
* ``gllm/model/transformer.py:45-78`` — pre-norm residual block.
* ``gllm/model/layers/norm.py:15-22`` — RMSNorm ``(x / sqrt(mean(x^2)+eps)) * w``.
* ``gllm/model/layers/mlp.py:44-47`` — ``down(silu(gate(x)) * up(x))``.
* ``gllm/model/layers/attention.py:122-182`` — projections around the hot path.
* ``gllm/llm/llm.py:145-348`` and ``gllm/engine/llm_engine.py:187-205`` —
  new-request prefill, one-token decode steps, block reservation on block
  boundaries, ``logits[arange, query_lens - 1]``.
* ``gllm/sample/sampler.py:67-106`` with ``top_k = 1`` — greedy argmax.

Only the path where every request finishes at the same step is restated
(requests never change batch index), which is what config (a) exercises.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch
import torch.nn.functional as F

from .attention import attention_layer_forward
from .metadata import BlockAllocator, Metadata, build_metadata, num_required_blocks
from .rope import rope_cache


@dataclass
class LlamaShape:
    num_layers: int = 16
    hidden: int = 2048
    num_q_heads: int = 32
    num_kv_heads: int = 8
    head_dim: int = 64
    ffn: int = 8192
    vocab: int = 128256
    rope_theta: float = 500000.0
    rms_eps: float = 1e-5


def init_weights(shape: LlamaShape, seed: int = 3, dtype=torch.float32) -> dict:
    """Random-init weights: N(0, 0.02) for every matrix, norms = 1."""
    g = torch.Generator().manual_seed(seed)
    H, D = shape.hidden, shape.head_dim
    kvd = shape.num_kv_heads * D

    def n(*s):
        return (torch.randn(*s, generator=g) * 0.02).to(dtype)

    w = {"embed": n(shape.vocab, H), "final_norm": torch.ones(H, dtype=dtype), "layers": []}
    for _ in range(shape.num_layers):
        w["layers"].append({
            "in_norm": torch.ones(H, dtype=dtype), "post_norm": torch.ones(H, dtype=dtype),
            "wq": n(shape.num_q_heads * D, H), "wk": n(kvd, H), "wv": n(kvd, H),
            "wo": n(H, shape.num_q_heads * D),
            "gate": n(shape.ffn, H), "up": n(shape.ffn, H), "down": n(H, shape.ffn),
        })
    return w


def rms_norm(x, w, eps):
    """``norm.py:15-22``."""
    ms = torch.mean(x * x, -1, keepdim=True)
    return (x / torch.sqrt(ms + eps)) * w


def mlp(x, lw):
    """``mlp.py:44-47``."""
    return F.linear(F.silu(F.linear(x, lw["gate"])) * F.linear(x, lw["up"]), lw["down"])


@dataclass
class StepRecord:
    meta: Metadata
    token_ids: torch.Tensor                 # [B, T_q] model input ids
    attn_out: list = field(default_factory=list)   # per layer [B, T_q, Hq, D]
    sampled: list = field(default_factory=list)


class OracleEngine:
    """CPU restatement of the engine loop over a fixed batch of prompts."""

    def __init__(self, shape: LlamaShape, weights: dict, block_size: int, max_batch: int,
                 max_seq_len: int, pad_token_id: int, dtype=torch.float32):
        self.s = shape
        self.w = weights
        self.bs = block_size
        self.max_seq_len = max_seq_len
        self.dtype = dtype
        self.pad = pad_token_id
        nb = num_required_blocks(max_batch * max_seq_len, block_size)  # paged_kv_cache.py:30
        self.num_blocks = nb
        self.k_cache = torch.zeros((shape.num_layers, nb * block_size, shape.num_kv_heads,
                                    shape.head_dim), dtype=dtype)
        self.v_cache = torch.zeros_like(self.k_cache)
        self.alloc = BlockAllocator(nb)
        self.cos, self.sin = rope_cache(max_seq_len, shape.head_dim, shape.rope_theta, dtype)
        self.width = num_required_blocks(max_seq_len, block_size)     # llm.py:44
        self.block_table = np.zeros((max_batch, self.width), dtype=np.int32)

    def forward(self, token_ids: torch.Tensor, meta: Metadata, rec: StepRecord | None):
        """``model.py:185-229`` + ``transformer.py:45-78`` + ``attention.py:122-182``."""
        s = self.s
        B, Tq = token_ids.shape
        x = self.w["embed"][token_ids]
        cos = self.cos[meta.positions]
        sin = self.sin[meta.positions]
        residual = None
        for li, lw in enumerate(self.w["layers"]):
            if residual is not None:
                x = x + residual
            residual = x
            h = rms_norm(x, lw["in_norm"], s.rms_eps)
            q = F.linear(h, lw["wq"]).view(B, Tq, s.num_q_heads, s.head_dim)
            k = F.linear(h, lw["wk"]).view(B, Tq, s.num_kv_heads, s.head_dim)
            v = F.linear(h, lw["wv"]).view(B, Tq, s.num_kv_heads, s.head_dim)
            a, _, _ = attention_layer_forward(q, k, v, cos, sin, self.k_cache[li],
                                              self.v_cache[li], meta)
            if rec is not None:
                rec.attn_out.append(a.clone())
            x = F.linear(a.reshape(B, Tq, -1), lw["wo"])
            x = x + residual
            residual = x
            x = mlp(rms_norm(x, lw["post_norm"], s.rms_eps), lw)
        return rms_norm(x + residual, self.w["final_norm"], s.rms_eps)

    def generate(self, prompts: list[list[int]], max_new_tokens: int,
                 record_steps: int | None = None):
        """Greedy generation; every request gets ``max_new_tokens`` tokens
        (no stop ids).  Returns (tokens per request, list of StepRecord)."""
        B = len(prompts)
        gen = [[] for _ in range(B)]
        nblocks = [0] * B
        records = []
        for step in range(max_new_tokens):
            if step == 0:
                ctx = [0] * B
                qlen = [len(p) for p in prompts]
                for i, p in enumerate(prompts):
                    n = num_required_blocks(len(p), self.bs)
                    self.block_table[i, :] = 0
                    self.block_table[i, :n] = self.alloc.reserve(n)
                    nblocks[i] = n
            else:
                ctx, qlen = [], []
                for i, p in enumerate(prompts):
                    L = len(p) + len(gen[i])
                    need = num_required_blocks(L, self.bs)
                    if need > nblocks[i]:
                        self.block_table[i, nblocks[i]:need] = self.alloc.reserve(need - nblocks[i])
                        nblocks[i] = need
                    ctx.append(L - 1)
                    qlen.append(1)
            meta = build_metadata(ctx, qlen, self.block_table, self.bs, self.dtype)
            Tq = max(qlen)
            ids = torch.full((B, Tq), self.pad, dtype=torch.int64)
            for i, p in enumerate(prompts):
                seq = p + gen[i]
                for r in range(qlen[i]):
                    ids[i, r] = seq[ctx[i] + r]
            rec = StepRecord(meta=meta, token_ids=ids) if (record_steps is None or step < record_steps) else None
            hs = self.forward(ids, meta, rec)
            logits = F.linear(hs, self.w["embed"])                      # model.py:232-239
            last = logits[torch.arange(B), meta.query_lens.to(torch.int64) - 1]   # llm.py:340
            tok = torch.argmax(last.to(torch.float32), dim=-1).tolist()  # sampler, top_k = 1
            for i in range(B):
                gen[i].append(tok[i])
            if rec is not None:
                rec.sampled = tok
                records.append(rec)
            if record_steps is not None and step + 1 >= record_steps:
                break
        return gen, records
