"""HIP graph capture of the attention launch, the way a serving loop runs a
decode step: capture once, replay every step.  The launch path only
enqueues kernels (no memset node, no allocation, no host wait), so it can be
captured.  Each replay must equal the eager result bit for bit (same
kernels, same inputs), with eager work and synchronisations between the
replays, and the eager result is itself checked against the CPU oracle."""
import pytest
import torch

from gllm_amd import paged
from tests.gpu_helpers import assert_close_bf16, make_batch, oracle_paged

pytestmark = pytest.mark.gpu

CASES = {
    # decode only, two heads per workgroup
    "decode": dict(ctx=[300, 17, 1500, 64, 900], ql=[1] * 5, Hq=32, Hkv=8, D=64, split=0),
    # decode with context splits (merge_splits_kernel runs in the graph too)
    "decode_split": dict(ctx=[4000, 33, 2500], ql=[1] * 3, Hq=64, Hkv=8, D=128, split=512),
    # page-balanced decode: split tickets drawn and re-armed inside the graph
    "decode_balanced": dict(ctx=[4000, 33, 2500, 700, 90], ql=[1] * 5, Hq=32, Hkv=8, D=64, split=paged.BALANCED),
    # mixed continuous batch: decodes plus two prefill chunks
    "mixed": dict(ctx=[700, 0, 250, 40], ql=[1, 90, 1, 33], Hq=32, Hkv=8, D=128, split=0),
}


@pytest.mark.parametrize("name", list(CASES))
def test_graph_replay_matches_eager(name):
    c = CASES[name]
    print(f"graph replay: {name}", flush=True)
    b = make_batch(c["ctx"], c["ql"], c["Hq"], c["Hkv"], c["D"])
    plan = paged.AttentionPlan(b.q_lens, b.seq_lens, num_q_heads=b.num_q_heads, num_kv_heads=b.num_kv_heads,
                               head_dim=b.head_dim, block_size=b.block_size, dtype=b.dtype, device="cuda",
                               split_tokens=c["split"])
    eager = paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table)
    torch.cuda.synchronize()
    assert_close_bf16(eager[: b.rows], oracle_paged(b), f"{name} eager")

    out = torch.empty_like(eager)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):                     # warm-up outside capture
        paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table, out=out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        paged.paged_attention(plan, b.q, b.k_cache, b.v_cache, b.block_table, out=out)
    for rep in range(4):
        out.fill_(float("nan"))                       # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out[: b.rows].view(torch.int16), eager[: b.rows].view(torch.int16)), f"{name} replay {rep}"
