"""Seeded synthetic inputs for the benchmark configurations.

Conventions: CPU ``torch.Generator`` seeds 0 (lengths), 1 (block tables) and
2 (values); values are N(0, 1) drawn in fp32 and cast to the model dtype;
block tables are slices of one ``randperm`` of ``[1, NB)`` (block 0 is the
reserved dummy).  Pools too large to draw on the host (configs d and e) draw
their values on the device from a seeded ``torch.Generator`` there instead.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch


@dataclass
class PagedBatch:
    name: str
    ctx_lens: list[int]
    q_lens: list[int]
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    num_blocks: int
    dtype: torch.dtype
    rope_theta: float | None = None
    kv_dtype: torch.dtype | None = None      # KV cache dtype (None: the model dtype)
    # filled by materialize()
    q: torch.Tensor | None = None            # [rows, Hq, D] (packed rows)
    k_new: torch.Tensor | None = None        # [rows, Hkv, D] new tokens' K (pre-RoPE)
    v_new: torch.Tensor | None = None
    k_cache: torch.Tensor | None = None      # [NB * bs, Hkv, D]
    v_cache: torch.Tensor | None = None
    block_table: torch.Tensor | None = None  # [B, W] int32
    slot_mapping: torch.Tensor | None = None # [rows] int64 slots of the new tokens
    q_row_start: list[int] = field(default_factory=list)
    cos: torch.Tensor | None = None          # [max_pos, D/2] table
    sin: torch.Tensor | None = None

    @property
    def seq_lens(self) -> list[int]:
        return [c + q for c, q in zip(self.ctx_lens, self.q_lens)]

    @property
    def rows(self) -> int:
        return sum(self.q_lens)

    def kv_bytes_per_token(self) -> int:
        kv = self.kv_dtype or self.dtype
        return 2 * self.num_kv_heads * self.head_dim * kv.itemsize


def block_tables(seq_lens, block_size, num_blocks, seed=1):
    g = torch.Generator().manual_seed(seed)
    need = [-(-L // block_size) for L in seq_lens]
    if sum(need) > num_blocks - 1:
        raise ValueError("pool too small")
    perm = torch.randperm(num_blocks - 1, generator=g).to(torch.int32) + 1
    W = max(need)
    bt = torch.zeros((len(seq_lens), W), dtype=torch.int32)
    o = 0
    for i, n in enumerate(need):
        bt[i, :n] = perm[o:o + n]
        o += n
    return bt


def materialize(b: PagedBatch, device, values_on_device: bool = False, seed: int = 2) -> PagedBatch:
    """Draw Q, new K/V and the pool contents; build tables and slots."""
    from .kv_cache import PagedKVCache  # noqa: F401  (layout documented there)
    Hq, Hkv, D = b.num_q_heads, b.num_kv_heads, b.head_dim
    rows = b.rows
    nslots = b.num_blocks * b.block_size
    bt = block_tables(b.seq_lens, b.block_size, b.num_blocks)
    if values_on_device:
        g = torch.Generator(device=device).manual_seed(seed)
        mk = lambda *s: torch.randn(*s, generator=g, device=device, dtype=torch.float32).to(b.dtype)
        b.q, b.k_new, b.v_new = mk(rows, Hq, D), mk(rows, Hkv, D), mk(rows, Hkv, D)
        b.k_cache = torch.empty(nslots, Hkv, D, dtype=b.dtype, device=device)
        b.v_cache = torch.empty(nslots, Hkv, D, dtype=b.dtype, device=device)
        chunk = 1 << 24
        for t in (b.k_cache, b.v_cache):
            flat = t.view(-1)
            for o in range(0, flat.numel(), chunk):
                n = min(chunk, flat.numel() - o)
                flat[o:o + n] = torch.randn(n, generator=g, device=device, dtype=torch.float32).to(b.dtype)
    else:
        g = torch.Generator().manual_seed(seed)
        mk = lambda *s: torch.randn(*s, generator=g, dtype=torch.float32).to(b.dtype)
        b.q, b.k_new, b.v_new = mk(rows, Hq, D), mk(rows, Hkv, D), mk(rows, Hkv, D)
        b.k_cache, b.v_cache = mk(nslots, Hkv, D), mk(nslots, Hkv, D)
        b.q, b.k_new, b.v_new = b.q.to(device), b.k_new.to(device), b.v_new.to(device)
        b.k_cache, b.v_cache = b.k_cache.to(device), b.v_cache.to(device)
    if b.kv_dtype is not None and b.kv_dtype != b.dtype:      # e.g. an fp8 pool: torch's cast of the draws
        b.k_cache, b.v_cache = b.k_cache.to(b.kv_dtype), b.v_cache.to(b.kv_dtype)
    b.block_table = bt.to(device)
    starts, slots = [], []
    r = 0
    for i, (c, q) in enumerate(zip(b.ctx_lens, b.q_lens)):
        starts.append(r)
        r += q
        p = torch.arange(c, c + q)
        slots.append(bt[i, p // b.block_size].to(torch.int64) * b.block_size + p % b.block_size)
    b.q_row_start = starts
    b.slot_mapping = torch.cat(slots).to(device)
    if b.rope_theta is not None:
        maxpos = max(b.seq_lens)
        p = torch.arange(maxpos)
        m = torch.arange(D // 2)
        ang = p.unsqueeze(1) * (b.rope_theta ** (-2 * m / D))
        b.cos = torch.cos(ang).to(b.dtype).to(device)
        b.sin = torch.sin(ang).to(b.dtype).to(device)
    return b


# ------------------------------------------------------------------ configs
def config_b() -> PagedBatch:
    """Decode, Llama-3.2-1B heads: B 64, 32/8 heads, D 64, L ~ U{128..2048}."""
    g = torch.Generator().manual_seed(0)
    L = torch.randint(128, 2049, (64,), generator=g).tolist()
    return PagedBatch("decode_1b", [x - 1 for x in L], [1] * 64, 32, 8, 64, 16, 16384, torch.bfloat16)


def config_c() -> PagedBatch:
    """Causal prefill + RoPE/KV write, Llama-3.1-8B heads: B 8, 32/8, D 128,
    prompt lengths ~ U{512..4096}, theta 5e5."""
    g = torch.Generator().manual_seed(0)
    L = torch.randint(512, 4097, (8,), generator=g).tolist()
    nb = sum(-(-x // 16) for x in L) + 1
    return PagedBatch("prefill_8b", [0] * 8, L, 32, 8, 128, 16, nb, torch.bfloat16, rope_theta=500000.0)


def config_d() -> PagedBatch:
    """Mixed batch, 8B heads: 256 decodes with L log-uniform in [256, 8192]
    plus 4 chunked prefills of 512 tokens on contexts ~ U{0..4096}; pool of
    131072 blocks."""
    g = torch.Generator().manual_seed(0)
    u = torch.rand(256, generator=g, dtype=torch.float64)
    Ld = [int(round(math.exp(math.log(256) + x * (math.log(8192) - math.log(256))))) for x in u.tolist()]
    cp = torch.randint(0, 4097, (4,), generator=g).tolist()
    ctx = [x - 1 for x in Ld] + cp
    ql = [1] * 256 + [512] * 4
    return PagedBatch("mixed_8b", ctx, ql, 32, 8, 128, 16, 131072, torch.bfloat16, rope_theta=500000.0)


def config_e() -> PagedBatch:
    """Long-context decode, Llama-3.1-70B heads (one GPU's share): B 128,
    64/8 heads, D 128, L ~ U{16384..32768}."""
    g = torch.Generator().manual_seed(0)
    L = torch.randint(16384, 32769, (128,), generator=g).tolist()
    nb = sum(-(-x // 16) for x in L) + 1
    return PagedBatch("long_decode_70b", [x - 1 for x in L], [1] * 128, 64, 8, 128, 16, nb, torch.bfloat16)


# ------------------------------------------------------------------ work
def decode_bytes(b: PagedBatch) -> int:
    """Compulsory HBM bytes of one attention launch over the batch: every
    sequence's K/V once, q and out once, block-table entries and lengths."""
    e = torch.finfo(b.dtype).bits // 8
    kv = sum(b.seq_lens) * b.kv_bytes_per_token()
    qo = 2 * b.rows * b.num_q_heads * b.head_dim * e
    bt = sum(-(-L // b.block_size) for L in b.seq_lens) * 4
    return kv + qo + bt + 8 * len(b.q_lens)


def attention_flops(b: PagedBatch) -> int:
    """Useful (unmasked) flops: 4 * Hq * D * (q*c + q(q+1)/2) per sequence."""
    return sum(4 * b.num_q_heads * b.head_dim * (q * c + q * (q + 1) // 2)
               for c, q in zip(b.ctx_lens, b.q_lens))


def rope_write_bytes(b: PagedBatch) -> int:
    """RoPE + KV write: read new K/V, write them to the pool, read cos/sin."""
    e = torch.finfo(b.dtype).bits // 8
    return b.rows * (2 * b.num_kv_heads * b.head_dim * e * 2 + b.head_dim * e)
