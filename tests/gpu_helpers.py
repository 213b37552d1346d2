"""Shared helpers for the GPU parity tests (inputs on the CPU, oracle on the
CPU, product on the GPU)."""
from __future__ import annotations

import torch

from gllm_amd import workloads
from oracle import attention as oa

MAX_ABS = 2e-2   # bf16 output vs fp32 reference, the benchmark tolerance
MEAN_ABS = 2e-3


def assert_close_bf16(out: torch.Tensor, ref: torch.Tensor, what: str = "", max_abs: float = MAX_ABS):
    d = (out.float().cpu() - ref.float().cpu()).abs()
    assert torch.isfinite(out.float()).all(), f"{what}: non-finite output"
    mx, mean = d.max().item(), d.mean().item()
    assert mx <= max_abs and mean <= MEAN_ABS, f"{what}: max-abs {mx:.3e} mean-abs {mean:.3e}"
    return mx, mean


def make_batch(ctx, ql, Hq, Hkv, D, bs=16, num_blocks=None, dtype=torch.bfloat16, theta=None, device="cuda"):
    seq = [c + q for c, q in zip(ctx, ql)]
    nb = num_blocks or (sum(-(-L // bs) for L in seq) * 2 + 8)
    b = workloads.PagedBatch("t", list(ctx), list(ql), Hq, Hkv, D, bs, nb, dtype, rope_theta=theta)
    return workloads.materialize(b, device)


def oracle_paged(b: workloads.PagedBatch, q_rot: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 reference for every real row of the batch (CPU)."""
    q = (q_rot if q_rot is not None else b.q).cpu()
    return oa.paged_attention(q, b.k_cache.cpu(), b.v_cache.cpu(), b.block_table.cpu(), b.ctx_lens,
                              b.q_lens, b.q_row_start, b.block_size)
