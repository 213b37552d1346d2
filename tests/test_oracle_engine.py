"""Pins the oracle engine (paged KV cache, left-padded metadata, prefill then
one-token decode steps) against a cache-free full recompute: at every step,
running the whole sequence through a plain causal transformer must give the
same greedy token.  A wrong slot, pad side, position or RoPE row in the
paged path changes the logits and fails this."""
import torch
import torch.nn.functional as F

from oracle.engine import LlamaShape, OracleEngine, init_weights, mlp, rms_norm
from oracle.rope import apply_rope, rope_cache


def _full_forward(shape, w, ids):
    """Textbook causal forward of one sequence (no cache, no padding)."""
    T = len(ids)
    x = w["embed"][torch.tensor(ids)].unsqueeze(0)
    cos, sin = rope_cache(T, shape.head_dim, shape.rope_theta, torch.float32)
    pos = torch.arange(T).unsqueeze(0)
    G = shape.num_q_heads // shape.num_kv_heads
    for lw in w["layers"]:
        h = rms_norm(x, lw["in_norm"], shape.rms_eps)
        q = F.linear(h, lw["wq"]).view(1, T, shape.num_q_heads, shape.head_dim)
        k = F.linear(h, lw["wk"]).view(1, T, shape.num_kv_heads, shape.head_dim)
        v = F.linear(h, lw["wv"]).view(1, T, shape.num_kv_heads, shape.head_dim)
        q = apply_rope(q, cos[pos], sin[pos])
        k = apply_rope(k, cos[pos], sin[pos])
        k = torch.repeat_interleave(k, G, dim=2)
        v = torch.repeat_interleave(v, G, dim=2)
        a = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), is_causal=True)
        x = x + F.linear(a.transpose(1, 2).reshape(1, T, -1), lw["wo"])
        x = x + mlp(rms_norm(x, lw["post_norm"], shape.rms_eps), lw)
    return F.linear(rms_norm(x, w["final_norm"], shape.rms_eps), w["embed"])[0, -1]


def test_oracle_engine_matches_full_recompute():
    shape = LlamaShape(num_layers=2, hidden=64, num_q_heads=4, num_kv_heads=2, head_dim=16, ffn=128,
                       vocab=300, rope_theta=10000.0)
    w = init_weights(shape, seed=5)
    for lw in w["layers"]:                       # larger weights: sharper, tie-free logits
        for k in ("wq", "wk", "wv", "wo", "gate", "up", "down"):
            lw[k] *= 20.0
    w["embed"] *= 20.0
    g = torch.Generator().manual_seed(6)
    prompts = [torch.randint(0, 300, (L,), generator=g).tolist() for L in (5, 17, 3, 11)]
    eng = OracleEngine(shape, w, block_size=4, max_batch=4, max_seq_len=48, pad_token_id=299)
    toks, _ = eng.generate(prompts, 12)
    for i, p in enumerate(prompts):
        seq = list(p)
        for t in range(12):
            logits = _full_forward(shape, w, seq)
            assert int(torch.argmax(logits)) == toks[i][t], (i, t)
            seq.append(toks[i][t])
