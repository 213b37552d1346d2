"""GPU engine slice for benchmark config (a): the Llama-shaped model of
``oracle.engine`` run on the GPU, with the attention hot path on the product
(``gllm_amd.Attention`` + ``PagedKVCache``) and plain torch for the
projections, norms, MLP and logits (outside the hot path).

Batch metadata comes from the host restatement of ``LLM.prepare_batch``
(``oracle.metadata``), i.e. what the reference engine would hand the
attention layer; it is an input to the product, not part of it.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

import gllm_amd
from oracle.engine import LlamaShape, mlp, rms_norm
from oracle.metadata import BlockAllocator, build_metadata, num_required_blocks
from oracle.rope import rope_cache


class _Cfg:
    def __init__(self, s: LlamaShape, dtype):
        self.num_attn_heads = s.num_q_heads
        self.num_kv_heads = s.num_kv_heads
        self.head_dim = s.head_dim
        self.hidden_size = s.num_q_heads * s.head_dim
        self.dtype = dtype


class GpuEngineSlice:
    def __init__(self, shape: LlamaShape, weights: dict, block_size: int, max_batch: int, max_seq_len: int,
                 pad_token_id: int, device="cuda", dtype=torch.float32):
        self.s = shape
        self.dev = torch.device(device)
        self.bs = block_size
        self.dtype = dtype
        self.pad = pad_token_id
        mv = lambda t: t.to(self.dev, dtype)
        self.embed = mv(weights["embed"])
        self.final_norm = mv(weights["final_norm"])
        self.layers = []
        cfg = _Cfg(shape, dtype)
        for li, lw in enumerate(weights["layers"]):
            pre = f"model.layers.{li}.self_attn"
            att = gllm_amd.Attention(li, cfg, {f"{pre}.q_proj.weight": lw["wq"], f"{pre}.k_proj.weight": lw["wk"],
                                               f"{pre}.v_proj.weight": lw["wv"], f"{pre}.o_proj.weight": lw["wo"]})
            att.W_q, att.W_k, att.W_v, att.W_o = mv(lw["wq"]), mv(lw["wk"]), mv(lw["wv"]), mv(lw["wo"])
            self.layers.append({"att": att, "in_norm": mv(lw["in_norm"]), "post_norm": mv(lw["post_norm"]),
                                "gate": mv(lw["gate"]), "up": mv(lw["up"]), "down": mv(lw["down"])})
        self.cache = gllm_amd.PagedKVCache(shape.num_layers, shape.num_kv_heads, shape.head_dim, block_size,
                                           max_batch, max_seq_len, dtype, self.dev)
        self.alloc = BlockAllocator(self.cache.num_blocks)
        cos, sin = rope_cache(max_seq_len, shape.head_dim, shape.rope_theta, dtype)
        self.cos, self.sin = cos.to(self.dev), sin.to(self.dev)
        self.block_table = np.zeros((max_batch, num_required_blocks(max_seq_len, block_size)), dtype=np.int32)

    def forward(self, ids, meta, record):
        s = self.s
        B, Tq = ids.shape
        gm = gllm_amd.AttentionMetadata(
            query_lens=meta.query_lens.to(self.dev), seq_lens=meta.seq_lens.to(self.dev),
            max_seq_len=meta.max_seq_len, block_table=meta.block_table.to(self.dev),
            slot_mapping=meta.slot_mapping.to(self.dev), query_slot_mapping=meta.query_slot_mapping.to(self.dev),
            bias=None, block_size=self.bs)
        pos = meta.positions.to(self.dev)
        cos, sin = self.cos[pos], self.sin[pos]
        x = self.embed[ids.to(self.dev)]
        residual = None
        outs = []
        for li, L in enumerate(self.layers):
            if residual is not None:
                x = x + residual
            residual = x
            h = rms_norm(x, L["in_norm"], s.rms_eps)
            att = L["att"]
            q = F.linear(h, att.W_q).view(B, Tq, s.num_q_heads, s.head_dim)
            k = F.linear(h, att.W_k).view(B, Tq, s.num_kv_heads, s.head_dim)
            v = F.linear(h, att.W_v).view(B, Tq, s.num_kv_heads, s.head_dim)
            a = att.attention(q, k, v, cos, sin, self.cache.get_layer_kv_cache(li), gm)
            if record:
                outs.append(a.cpu())
            x = F.linear(a.reshape(B, Tq, -1), att.W_o) + residual
            residual = x
            x = mlp(rms_norm(x, L["post_norm"], s.rms_eps), L)
        hs = rms_norm(x + residual, self.final_norm, s.rms_eps)
        return hs, outs

    def generate(self, prompts, max_new_tokens, record_steps):
        B = len(prompts)
        gen = [[] for _ in range(B)]
        nblocks = [0] * B
        metas, att_outs = [], []
        for step in range(max_new_tokens):
            if step == 0:
                ctx, qlen = [0] * B, [len(p) for p in prompts]
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
            hs, outs = self.forward(ids, meta, step < record_steps)
            logits = F.linear(hs, self.embed)
            last = logits[torch.arange(B, device=self.dev), meta.query_lens.to(self.dev).long() - 1]
            tok = torch.argmax(last.float(), dim=-1).tolist()
            for i in range(B):
                gen[i].append(tok[i])
            if step < record_steps:
                metas.append(meta)
                att_outs.append(outs)
        return gen, metas, att_outs
