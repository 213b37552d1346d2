"""benchmark config (a): a random-init Llama-3.2-1B-shaped model (16 layers,
hidden 2048, 32/8 heads, head_dim 64, FFN 8192, vocab 128256, RoPE theta
5e5, fp32 weights from seed 3) through the reference's batching path: 8
prompts of uniform-random ids (lengths U{8..64}, seed 4), greedy decode of
64 new tokens, block_size 16, max_batch 8, max_seq_len 256.

The CPU oracle engine (restatement of the reference engine) runs the first
16 steps; the GPU engine slice (product attention hot path) runs all 64.
Checks: every recorded step's per-layer attention output on real rows within
fp32 tolerance, and the first 16 generated tokens equal.
"""
import pytest
import torch

from oracle.engine import LlamaShape, OracleEngine, init_weights
from tests.engine_slice import GpuEngineSlice

pytestmark = pytest.mark.gpu

PAD = 128001          # first eos id of Llama-3.2-1B-Instruct, the reference's pad_token_id
STEPS_CHECKED = 16


@pytest.mark.timeout(600)
def test_config_a_engine_parity():
    print("config (a): building weights", flush=True)
    torch.set_num_threads(max(1, min(16, torch.get_num_threads())))
    shape = LlamaShape()
    weights = init_weights(shape, seed=3)
    g = torch.Generator().manual_seed(4)
    lens = torch.randint(8, 65, (8,), generator=g).tolist()
    prompts = [torch.randint(0, 128000, (L,), generator=g).tolist() for L in lens]

    print("config (a): GPU engine slice, 64 tokens", flush=True)
    gpu = GpuEngineSlice(shape, weights, block_size=16, max_batch=8, max_seq_len=256, pad_token_id=PAD)
    gtok, gmetas, gouts = gpu.generate(prompts, 64, record_steps=STEPS_CHECKED)
    assert all(len(t) == 64 for t in gtok)
    del gpu
    torch.cuda.empty_cache()

    print("config (a): CPU oracle engine, 16 tokens", flush=True)
    ora = OracleEngine(shape, weights, block_size=16, max_batch=8, max_seq_len=256, pad_token_id=PAD)
    otok, recs = ora.generate(prompts, STEPS_CHECKED, record_steps=STEPS_CHECKED)

    worst = 0.0
    for step, rec in enumerate(recs):
        m = rec.meta
        assert torch.equal(m.slot_mapping, gmetas[step].slot_mapping)
        ql = m.query_lens.tolist()
        for li in range(shape.num_layers):
            ref, out = rec.attn_out[li], gouts[step][li]
            for i, q in enumerate(ql):
                d = (out[i, :q] - ref[i, :q]).abs()
                worst = max(worst, d.max().item())
                assert d.max().item() < 1e-3 and d.mean().item() < 1e-4, (step, li, i, d.max().item())
    print(f"config (a): worst per-layer attention max-abs diff {worst:.3e}", flush=True)
    for i in range(8):
        assert gtok[i][:STEPS_CHECKED] == otok[i][:STEPS_CHECKED], (i, gtok[i][:STEPS_CHECKED], otok[i])
