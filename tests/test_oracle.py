"""Pins the CPU oracle against closed forms, brute force and invariants.

The reference ships no golden vectors for this path, so each oracle function
is checked here against what the mathematics fixes, chosen so that a plausible
slip (wrong half pairing, wrong GQA index, dropped scale, off-by-one in the
mask, wrong padding side) fails at least one test.
"""
import itertools
import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import bruteforce as bf
from oracle import metadata as om
from oracle import rope as orope


# ---------------------------------------------------------------- metadata
def _tiny_batch(seed, B=3, bs=4, nb=40):
    g = torch.Generator().manual_seed(seed)
    ctx = torch.randint(0, 9, (B,), generator=g).tolist()
    q = torch.randint(1, 6, (B,), generator=g).tolist()
    bt = om.random_block_tables([c + n for c, n in zip(ctx, q)], bs, nb, g, width=8)
    return ctx, q, bt, bs


@pytest.mark.parametrize("seed", range(6))
def test_metadata_bruteforce(seed):
    ctx, q, bt, bs = _tiny_batch(seed)
    m = om.build_metadata(ctx, q, bt, bs)
    B = len(q)
    max_ctx, max_q = max(ctx), max(q)
    T = max_ctx + max_q
    assert m.slot_mapping.shape == (B, T) and m.bias.shape == (B, max_q, T)
    for i in range(B):
        pad = max_ctx - ctx[i]
        L = ctx[i] + q[i]
        for j in range(T):
            p = j - pad
            want_slot = om.slot_of(bt[i], p, bs) if 0 <= p < L else 0
            assert int(m.slot_mapping[i, j]) == want_slot
            for r in range(max_q):
                # element-wise restatement of llm.py:264-274
                if j < pad:
                    want = -math.inf
                elif j < max_ctx:
                    want = 0.0
                else:
                    want = 0.0 if (j - max_ctx) <= r else -math.inf
                assert float(m.bias[i, r, j]) == want
                # mask-equivalence theorem on real rows: visible <=> p <= c+r
                if r < q[i] and 0 <= p < L:
                    assert (want == 0.0) == (p <= ctx[i] + r)
                if r < q[i] and not (0 <= p < L):
                    assert want == -math.inf
        for r in range(max_q):
            # llm.py:281 on real rows; padded rows clamped to the last real position
            assert int(m.positions[i, r]) == (ctx[i] + r if r < q[i] else L - 1)
            want = om.slot_of(bt[i], ctx[i] + r, bs) if r < q[i] else 0
            assert int(m.query_slot_mapping[i, r]) == want


def test_padded_positions_stay_inside_the_rope_table():
    # a mixed batch: decode rows padded to the prefill chunk's T_q.  llm.py:281
    # would give the decode rows positions up to c_i + T_q - 1 (past the end of
    # a max_seq_len-row RoPE table); the clamp keeps every position < max L_i
    ctx, ql, bs = [8000, 100, 3000], [1, 512, 1], 16
    max_seq_len = max(c + q for c, q in zip(ctx, ql))           # 8001 rows of cos/sin
    g = torch.Generator().manual_seed(5)
    bt = om.random_block_tables([c + q for c, q in zip(ctx, ql)], bs, 1200, g)
    m = om.build_metadata(ctx, ql, bt, bs)
    assert ctx[0] + max(ql) - 1 >= max_seq_len                   # the unclamped value would overflow
    assert int(m.positions.max()) == max_seq_len - 1
    assert m.positions[0].tolist() == [8000] * 512               # decode row 0 real, rows 1.. padded
    assert m.positions[1].tolist() == list(range(100, 612))      # the chunk: all real
    assert m.positions[2].tolist() == [3000] * 512
    cos = torch.randn(max_seq_len, 32)
    assert cos[m.positions].shape == (3, 512, 32)                # model.py:195's gather is in range


def test_metadata_invariants():
    g = torch.Generator().manual_seed(11)
    lens = torch.randint(1, 200, (16,), generator=g).tolist()
    bt = om.random_block_tables(lens, 16, 1024, g)
    m = om.build_metadata([L - 1 for L in lens], [1] * 16, bt, 16)
    live = [int(m.slot_mapping[i, j]) for i in range(16) for j in range(m.slot_mapping.shape[1])
            if float(m.bias[i, 0, j]) == 0.0]
    assert len(live) == len(set(live)) == sum(lens)
    assert all(16 <= s < 1024 * 16 for s in live)       # block 0 never live
    assert m.query_slot_mapping.shape == (16, 1)


def test_allocator_semantics():
    a = om.BlockAllocator(6)
    assert a.reserve(2) == [5, 4]
    a.release([5])
    assert a.reserve(3) == [3, 2, 1]
    assert 5 in a.cached
    with pytest.raises(TypeError):
        a.reserve(1)        # free list empty: dict.pop() without a key raises, as the reference
    assert om.num_required_blocks(16, 16) == 1 and om.num_required_blocks(17, 16) == 2


# ---------------------------------------------------------------- RoPE
def test_rope_table_closed_form():
    cos, sin = orope.rope_cache(64, 64, 500000.0, torch.float32)
    assert torch.equal(cos[0], torch.ones(32)) and torch.equal(sin[0], torch.zeros(32))
    for p in (1, 7, 63):
        for j in (0, 5, 31):
            a = p * 500000.0 ** (-2 * j / 64)
            assert abs(float(cos[p, j]) - math.cos(a)) < 1e-5
            assert abs(float(sin[p, j]) - math.sin(a)) < 1e-5
    cb, sb = orope.rope_cache(64, 64, 500000.0, torch.bfloat16)
    assert torch.equal(cb, cos.to(torch.bfloat16)) and torch.equal(sb, sin.to(torch.bfloat16))


def test_rope_known_answers():
    D = 8
    x = torch.zeros(1, 1, 1, D)
    x[..., 0] = 1.0                                   # pair (x_0, x_4) = (1, 0)
    c = torch.zeros(1, 1, D // 2)
    s = torch.zeros(1, 1, D // 2)
    c[..., 0], s[..., 0] = 0.0, 1.0                   # 90 degrees
    out = orope.apply_rope(x, c, s)
    assert float(out[..., 0]) == 0.0 and float(out[..., 4]) == 1.0   # (1,0) -> (0,1)
    x2 = torch.zeros(1, 1, 1, D)
    x2[..., 4] = 1.0                                  # (0,1) -> (-1,0)
    out2 = orope.apply_rope(x2, c, s)
    assert float(out2[..., 0]) == -1.0 and float(out2[..., 4]) == 0.0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rope_properties(dtype):
    g = torch.Generator().manual_seed(5)
    D, theta = 64, 500000.0
    cos, sin = orope.rope_cache(128, D, theta, dtype)
    x = torch.randn(2, 5, 3, D, generator=g).to(dtype)
    pos = torch.tensor([[0, 1, 2, 50, 127], [3, 9, 64, 100, 0]])
    out = orope.apply_rope(x, cos[pos], sin[pos])
    # position 0 is the identity, exactly
    assert torch.equal(out[0, 0], x[0, 0]) and torch.equal(out[1, 4], x[1, 4])
    # pair norms preserved; fp64 closed form agrees
    tol = 1e-5 if dtype == torch.float32 else 3e-2
    x64 = x.double()
    o64 = out.double()
    h = D // 2
    n_in = x64[..., :h] ** 2 + x64[..., h:] ** 2
    n_out = o64[..., :h] ** 2 + o64[..., h:] ** 2
    assert torch.allclose(n_in, n_out, atol=tol * 10, rtol=tol * 10)
    for b, t in itertools.product(range(2), range(5)):
        ref = bf.rotate_fp64(x64[b, t].numpy(), int(pos[b, t]), theta)
        assert np.allclose(o64[b, t].numpy(), ref, atol=tol * 4, rtol=tol)
    if dtype == torch.float32:
        # inverse rotation (sin -> -sin) recovers the input
        back = orope.apply_rope(out, cos[pos], -sin[pos])
        assert torch.allclose(back, x, atol=1e-5)


# ---------------------------------------------------------------- attention op
@pytest.mark.parametrize("B,Tq,T,Hq,Hkv,D", [(1, 3, 5, 1, 1, 4), (2, 2, 6, 4, 2, 8), (1, 4, 7, 8, 2, 4)])
def test_reference_attention_bruteforce(B, Tq, T, Hq, Hkv, D):
    g = torch.Generator().manual_seed(B * 100 + T)
    q = torch.randn(B, Tq, Hq, D, generator=g)
    k = torch.randn(B, T, Hkv, D, generator=g)
    v = torch.randn(B, T, Hkv, D, generator=g)
    bias = torch.zeros(B, Tq, T)
    bias[:, :, T - Tq:] = torch.full((Tq, Tq), float("-inf")).triu(1)
    bias[0, 0, 0] = float("-inf")
    out = oa.reference_attention(q, k, v, bias)
    ref = bf.sdpa_fp64(q.numpy(), k.numpy(), v.numpy(), bias.numpy())
    assert np.allclose(out.numpy(), ref, atol=1e-5)


def test_reference_attention_special_cases():
    g = torch.Generator().manual_seed(1)
    B, Tq, T, Hq, Hkv, D = 1, 2, 5, 4, 2, 8
    q = torch.randn(B, Tq, Hq, D, generator=g)
    k = torch.randn(B, T, Hkv, D, generator=g)
    v = torch.randn(B, T, Hkv, D, generator=g)
    one = torch.full((B, Tq, T), float("-inf"))
    one[:, :, 3] = 0.0                               # exactly one visible key
    out = oa.reference_attention(q, k, v, one)
    for h in range(Hq):
        assert torch.allclose(out[0, :, h], v[0, 3, h // 2].expand(Tq, D), atol=1e-6)
    zq = torch.zeros_like(q)
    bias = torch.zeros(B, Tq, T)
    bias[:, :, 0] = float("-inf")
    out = oa.reference_attention(zq, k, v, bias)   # Q = 0 => mean of visible V
    for h in range(Hq):
        assert torch.allclose(out[0, 0, h], v[0, 1:, h // 2].mean(0), atol=1e-6)
    full = torch.full((B, Tq, T), float("-inf"))
    assert torch.isnan(oa.reference_attention(q, k, v, full)).all()


def test_gqa_head_mapping():
    # kv head j carries constant value j in V; q head h must read h // G
    B, Tq, T, Hq, Hkv, D = 1, 1, 3, 8, 2, 4
    q = torch.randn(B, Tq, Hq, D)
    k = torch.randn(B, T, Hkv, D)
    v = torch.stack([torch.full((B, T, D), float(j)) for j in range(Hkv)], dim=2)
    out = oa.reference_attention(q, k, v, torch.zeros(B, Tq, T))
    for h in range(Hq):
        assert torch.allclose(out[0, 0, h], torch.full((D,), float(h // 4)))


# ---------------------------------------------------------------- call site
def _layer_case(seed, dtype=torch.float32, bs=4):
    g = torch.Generator().manual_seed(seed)
    ctx, ql, bt, _ = _tiny_batch(seed, bs=bs)
    Hq, Hkv, D = 4, 2, 8
    meta = om.build_metadata(ctx, ql, bt, bs, dtype)
    B, Tq = meta.query_slot_mapping.shape
    nslots = 40 * bs
    kc = torch.randn(nslots, Hkv, D, generator=g).to(dtype)
    vc = torch.randn(nslots, Hkv, D, generator=g).to(dtype)
    q = torch.randn(B, Tq, Hq, D, generator=g).to(dtype)
    k = torch.randn(B, Tq, Hkv, D, generator=g).to(dtype)
    v = torch.randn(B, Tq, Hkv, D, generator=g).to(dtype)
    cos, sin = orope.rope_cache(64, D, 10000.0, dtype)
    return ctx, ql, bt, meta, kc, vc, q, k, v, cos[meta.positions], sin[meta.positions]


@pytest.mark.parametrize("seed", range(4))
def test_layer_write_then_gather_and_paged_equivalence(seed):
    ctx, ql, bt, meta, kc, vc, q, k, v, cos, sin = _layer_case(seed)
    kc0, vc0 = kc.clone(), vc.clone()
    out, qr, kr = oa.attention_layer_forward(q, k, v, cos, sin, kc, vc, meta)
    B, Tq = meta.query_slot_mapping.shape
    bs = 4
    written = set()
    for i in range(B):
        for r in range(ql[i]):
            s = int(meta.query_slot_mapping[i, r])
            written.add(s)
            assert torch.equal(kc[s], kr[i, r]) and torch.equal(vc[s], v[i, r])
    # sentinel: everything outside written slots and dummy block 0 unchanged
    for s in range(kc.shape[0]):
        if s not in written and s >= bs:
            assert torch.equal(kc[s], kc0[s]) and torch.equal(vc[s], vc0[s])
    # the paged per-sequence form equals the dense padded form on real rows
    rows = qr.reshape(B * Tq, *qr.shape[2:])
    po = oa.paged_attention(rows, kc, vc, torch.from_numpy(bt), ctx, ql,
                            [i * Tq for i in range(B)], bs)
    for i in range(B):
        assert torch.allclose(po[i * Tq:i * Tq + ql[i]], out[i, :ql[i]], atol=1e-5)


def test_paged_attention_bruteforce():
    ctx, ql, bt, meta, kc, vc, q, k, v, cos, sin = _layer_case(7)
    B, Tq = meta.query_slot_mapping.shape
    rows = q.reshape(B * Tq, *q.shape[2:])
    po = oa.paged_attention(rows, kc, vc, torch.from_numpy(bt), ctx, ql, [i * Tq for i in range(B)], 4)
    for i in range(B):
        L = ctx[i] + ql[i]
        slots = [om.slot_of(bt[i], p, 4) for p in range(L)]
        kk = kc[slots].unsqueeze(0).numpy()
        vv = vc[slots].unsqueeze(0).numpy()
        qq = q[i:i + 1, :ql[i]].numpy()
        bias = np.array([[0.0 if p <= ctx[i] + r else -np.inf for p in range(L)] for r in range(ql[i])])[None]
        ref = bf.sdpa_fp64(qq, kk, vv, bias)
        assert np.allclose(po[i * Tq:i * Tq + ql[i]].numpy(), ref[0], atol=1e-5)


def test_lse_split_merge_identity():
    g = torch.Generator().manual_seed(3)
    s = torch.randn(4, 37, generator=g) * 3
    v = torch.randn(37, 6, generator=g)
    full = torch.softmax(s, -1) @ v
    cuts = [0, 5, 17, 30, 37]
    ms, ls, accs = [], [], []
    for a, b in zip(cuts[:-1], cuts[1:]):
        m = s[:, a:b].max(-1).values
        e = torch.exp(s[:, a:b] - m.unsqueeze(-1))
        ms.append(m)
        ls.append(e.sum(-1))
        accs.append(e @ v[a:b])
    assert torch.allclose(oa.lse_merge(ms, ls, accs), full, atol=1e-6)


# ------------------------------------------------------------ fused projection (attention.py:139-161)
def test_oracle_linear_brute_force():
    """linear.py:13-19 (F.linear: x @ W^T, W [out, in]) on tiny inputs against
    Python-float dot products, rounded once to bf16."""
    from oracle import projection as op
    g = torch.Generator().manual_seed(5)
    x = torch.randn(3, 7, generator=g).to(torch.bfloat16)
    w = torch.randn(5, 7, generator=g).to(torch.bfloat16)
    got = op.linear(x, w)
    for i in range(3):
        for j in range(5):
            ref = sum(float(x[i, k]) * float(w[j, k]) for k in range(7))
            assert got[i, j].item() == torch.tensor(ref, dtype=torch.float64).to(torch.bfloat16).item()
    # fp32 inputs keep fp32 (the fp32 model path) and W is used transposed
    xf, wf = torch.randn(2, 4, generator=g), torch.randn(3, 4, generator=g)
    assert torch.allclose(op.linear(xf, wf), xf @ wf.t(), atol=1e-6)


def test_oracle_qkv_identity_rotation_and_padding():
    """Position 0 (cos 1, sin 0) leaves q/k unrotated, so the cache holds
    exactly the projections; rows marked padded leave a sentinel pool alone."""
    from oracle import projection as op
    g = torch.Generator().manual_seed(6)
    n, hidden, Hq, Hkv, D = 5, 32, 4, 2, 8
    x = torch.randn(n, hidden, generator=g).to(torch.bfloat16)
    wq = torch.randn(Hq * D, hidden, generator=g).to(torch.bfloat16)
    wk = torch.randn(Hkv * D, hidden, generator=g).to(torch.bfloat16)
    wv = torch.randn(Hkv * D, hidden, generator=g).to(torch.bfloat16)
    cos = torch.ones(n, D // 2, dtype=torch.bfloat16)
    sin = torch.zeros(n, D // 2, dtype=torch.bfloat16)
    kc = torch.full((20, Hkv, D), 7.0, dtype=torch.bfloat16)
    vc = kc.clone()
    slots = torch.tensor([3, 9, 0, 14, 11])
    real = torch.tensor([True, True, False, True, True])
    q = op.qkv_rope_kv_write(x, wq, wk, wv, cos, sin, kc, vc, slots, Hkv, D, real=real)
    assert torch.equal(q.reshape(n, -1), op.linear(x, wq))
    for t in (0, 1, 3, 4):
        assert torch.equal(kc[slots[t]].reshape(-1), op.linear(x[t:t + 1], wk)[0])
        assert torch.equal(vc[slots[t]].reshape(-1), op.linear(x[t:t + 1], wv)[0])
    untouched = [s for s in range(20) if s not in (3, 9, 14, 11)]
    assert torch.all(kc[untouched] == 7.0) and torch.all(vc[untouched] == 7.0)


def test_oracle_qkv_identity_projection_is_rope_write():
    """With identity projections (hidden = Hkv*D, W = I) the fused step is the
    plain RoPE + KV write, pinned on its own above (rotation known angles,
    write-then-gather round trip)."""
    from oracle import projection as op
    from oracle import attention as oa
    from oracle import rope as orope
    g = torch.Generator().manual_seed(7)
    n, Hkv, D = 6, 2, 16
    hidden = Hkv * D
    x = torch.randn(n, hidden, generator=g).to(torch.bfloat16)
    eye = torch.eye(hidden, dtype=torch.bfloat16)
    cos_t, sin_t = orope.rope_cache(32, D, 10000.0, torch.bfloat16)
    pos = torch.tensor([0, 5, 9, 17, 30, 2])
    kc = torch.zeros(10, Hkv, D, dtype=torch.bfloat16)
    vc = kc.clone()
    slots = torch.tensor([1, 2, 3, 4, 5, 6])
    q = op.qkv_rope_kv_write(x, eye, eye, eye, cos_t[pos], sin_t[pos], kc, vc, slots, Hkv, D)
    k_rot = orope.apply_rope(x.view(1, n, Hkv, D), cos_t[pos].unsqueeze(0), sin_t[pos].unsqueeze(0))[0]
    kc2, vc2 = torch.zeros_like(kc), torch.zeros_like(vc)
    oa.kv_write(kc2, vc2, slots, k_rot, x.view(n, Hkv, D))
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
    assert torch.equal(q, k_rot)


# ---------------------------------------------------------------- per-op rounding of apply_rope
def _bf16_rne(x: np.ndarray) -> np.ndarray:
    """fp32 -> nearest bf16 (ties to even), returned as fp32, from the bit
    pattern (NaN kept quiet)."""
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    r = np.where(nan, (u | 0x400000) & 0xFFFF0000, r)
    return r.astype(np.uint32).view(np.float32)


def test_apply_rope_bf16_rounds_after_every_op():
    """attention.py:105-118 in bf16 is six torch ops, each rounded to bf16:
    lo = r(r(x1 c) - r(x2 s)), hi = r(r(x1 s) + r(x2 c)).  A numpy brute force
    of exactly that (products exact in fp32, differences rounded to fp32 then
    to bf16) must equal the oracle bit for bit, and on the same inputs a
    single rounding of the exact result must differ often enough that the
    check tells the two apart."""
    g = torch.Generator().manual_seed(17)
    D = 128
    x = (torch.randn(4, 64, 2, D, generator=g) * 3).to(torch.bfloat16)
    cos_t, sin_t = orope.rope_cache(4096, D, 500000.0, torch.bfloat16)
    pos = torch.randint(0, 4096, (4, 64), generator=g)
    c, s = cos_t[pos], sin_t[pos]
    out = orope.apply_rope(x, c, s).float().numpy()
    xf = x.float().numpy()
    x1, x2 = xf[..., :D // 2], xf[..., D // 2:]
    cf = c.float().numpy()[:, :, None, :]
    sf = s.float().numpy()[:, :, None, :]
    lo = _bf16_rne(_bf16_rne(x1 * cf) - _bf16_rne(x2 * sf))
    hi = _bf16_rne(_bf16_rne(x1 * sf) + _bf16_rne(x2 * cf))
    want = np.concatenate([lo, hi], axis=-1)
    assert np.array_equal(out.view(np.uint32), want.view(np.uint32))
    x164, x264 = x1.astype(np.float64), x2.astype(np.float64)
    once = np.concatenate([_bf16_rne((x164 * cf - x264 * sf).astype(np.float32)),
                           _bf16_rne((x164 * sf + x264 * cf).astype(np.float32))], axis=-1)
    assert (once != want).mean() > 0.05


def test_apply_rope_fp32_has_no_fused_multiply_add():
    """In fp32 each product and the difference are rounded separately (torch
    runs them as separate ops): numpy float32 arithmetic reproduces it bit for
    bit, and a fused multiply-add or an fp64 evaluation would not."""
    g = torch.Generator().manual_seed(18)
    D = 64
    x = torch.randn(3, 40, 2, D, generator=g)
    cos_t, sin_t = orope.rope_cache(1000, D, 500000.0, torch.float32)
    pos = torch.randint(0, 1000, (3, 40), generator=g)
    c, s = cos_t[pos], sin_t[pos]
    out = orope.apply_rope(x, c, s).numpy()
    xf = x.numpy()
    x1, x2 = xf[..., :D // 2], xf[..., D // 2:]
    cf, sf = c.numpy()[:, :, None, :], s.numpy()[:, :, None, :]
    want = np.concatenate([x1 * cf - x2 * sf, x1 * sf + x2 * cf], axis=-1)
    assert np.array_equal(out.view(np.uint32), want.view(np.uint32))
    x164, x264 = x1.astype(np.float64), x2.astype(np.float64)
    exact = np.concatenate([(x164 * cf - x264 * sf), (x164 * sf + x264 * cf)], axis=-1).astype(np.float32)
    assert (exact != want).mean() > 0.01


# ---------------------------------------------------------------- RMSNorm / SiLU MLP (config (a)'s layer)
def test_rms_norm_properties():
    """norm.py:15-22: unit root-mean-square with unit weights, invariance to
    a positive scale (eps = 0), elementwise weight, one-hot closed form."""
    from oracle import engine as oe
    g = torch.Generator().manual_seed(19)
    x = torch.randn(5, 256, generator=g, dtype=torch.float64)
    ones = torch.ones(256, dtype=torch.float64)
    y = oe.rms_norm(x, ones, 0.0)
    assert torch.allclose((y * y).mean(-1), torch.ones(5, dtype=torch.float64), atol=1e-12)
    assert torch.allclose(oe.rms_norm(7.5 * x, ones, 0.0), y, atol=1e-12)
    w = torch.randn(256, generator=g, dtype=torch.float64)
    assert torch.allclose(oe.rms_norm(x, w, 0.0), y * w, atol=1e-12)
    e = torch.zeros(1, 256, dtype=torch.float64)
    e[0, 9] = -3.0
    oh = oe.rms_norm(e, ones, 0.0)
    assert abs(float(oh[0, 9]) + 16.0) < 1e-12 and float(oh.abs().sum()) == 16.0   # sqrt(256) * sign
    yeps = oe.rms_norm(e, ones, 1e-5)                                               # eps inside the root
    assert abs(float(yeps[0, 9]) + 3.0 / math.sqrt(9.0 / 256 + 1e-5)) < 1e-12


def test_silu_mlp_properties():
    """mlp.py:44-47, down(silu(gate x) * up x): with gate = up = down = I it is
    x * silu(x), checked at known values of silu; linear in down; zero when
    up = 0."""
    from oracle import engine as oe
    eye = torch.eye(4, dtype=torch.float64)
    lw = {"gate": eye, "up": eye, "down": eye}
    x = torch.tensor([[0.0, 1.0, -1.0, 2.0]], dtype=torch.float64)
    silu = [0.0, 0.7310585786300049, -0.2689414213699951, 1.7615941559557649]   # z / (1 + e^-z)
    want = torch.tensor([[xi * si for xi, si in zip([0.0, 1.0, -1.0, 2.0], silu)]], dtype=torch.float64)
    assert torch.allclose(oe.mlp(x, lw), want, atol=1e-14)
    g = torch.Generator().manual_seed(20)
    lw2 = {k: torch.randn(8, 8, generator=g, dtype=torch.float64) for k in ("gate", "up", "down")}
    xr = torch.randn(3, 8, generator=g, dtype=torch.float64)
    lw3 = dict(lw2, down=2.5 * lw2["down"])
    assert torch.allclose(oe.mlp(xr, lw3), 2.5 * oe.mlp(xr, lw2), atol=1e-12)
    assert torch.equal(oe.mlp(xr, dict(lw2, up=torch.zeros(8, 8, dtype=torch.float64))),
                       torch.zeros(3, 8, dtype=torch.float64))


def test_apply_rope_fp16_rounds_after_every_op():
    """attention.py:105-118 for an fp16 model: six torch ops, each rounded to
    fp16.  numpy float16 arithmetic (each op evaluated in float32 and rounded
    to float16, as torch's CPU half ops do) reproduces the oracle bit for
    bit; rounding only the exact result once differs often enough to tell
    the two apart."""
    g = torch.Generator().manual_seed(19)
    D = 64
    x = (torch.randn(3, 50, 2, D, generator=g) * 3).to(torch.float16)
    cos_t, sin_t = orope.rope_cache(4096, D, 500000.0, torch.float16)
    pos = torch.randint(0, 4096, (3, 50), generator=g)
    c, s = cos_t[pos], sin_t[pos]
    out = orope.apply_rope(x, c, s).numpy()
    xf = x.numpy()
    x1, x2 = xf[..., :D // 2], xf[..., D // 2:]
    cf, sf = c.numpy()[:, :, None, :], s.numpy()[:, :, None, :]
    want = np.concatenate([(x1 * cf) - (x2 * sf), (x1 * sf) + (x2 * cf)], axis=-1)
    assert want.dtype == np.float16
    assert np.array_equal(out.view(np.uint16), want.view(np.uint16))
    x164, x264 = x1.astype(np.float64), x2.astype(np.float64)
    c64, s64 = cf.astype(np.float64), sf.astype(np.float64)
    once = np.concatenate([x164 * c64 - x264 * s64, x164 * s64 + x264 * c64], axis=-1).astype(np.float16)
    assert (once != want).mean() > 0.05


@pytest.mark.parametrize("model,cache", [(torch.bfloat16, torch.float32), (torch.float16, torch.float32),
                                         (torch.bfloat16, torch.float16)])
def test_paged_attention_casts_the_gather_to_the_model_dtype(model, cache):
    """attention.py:169-170 gathers K/V with .to(q.dtype): a cache wider than
    (or other than) the model dtype is rounded to the model dtype before the
    attention.  The oracle's per-sequence form equals the reference's
    call-site path (attention_layer_forward: write, gather, dense SDPA in
    fp32) on such a cache, and the cast is visible: without it the result
    differs."""
    ctx, ql, bt, meta, kc, vc, q, k, v, cos, sin = _layer_case(3)
    g = torch.Generator().manual_seed(33)
    kc = torch.randn(kc.shape, generator=g).to(cache)
    vc = torch.randn(vc.shape, generator=g).to(cache)
    q, k, v = q.to(model), k.to(model), v.to(model)
    cos, sin = cos.to(model), sin.to(model)
    B, Tq = meta.query_slot_mapping.shape
    out, qr, _ = oa.attention_layer_forward(q, k, v, cos, sin, kc, vc, meta, sdpa_dtype=torch.float32)
    rows = qr.reshape(B * Tq, *qr.shape[2:])
    po = oa.paged_attention(rows, kc, vc, torch.from_numpy(bt), ctx, ql, [i * Tq for i in range(B)], 4)
    nocast = oa.paged_attention(rows.float(), kc.float(), vc.float(), torch.from_numpy(bt), ctx, ql,
                                [i * Tq for i in range(B)], 4)
    d_cast = d_nocast = 0.0
    for i in range(B):
        d_cast = max(d_cast, (po[i * Tq:i * Tq + ql[i]] - out[i, :ql[i]].float()).abs().max().item())
        d_nocast = max(d_nocast, (nocast[i * Tq:i * Tq + ql[i]] - out[i, :ql[i]].float()).abs().max().item())
    assert d_cast < 1e-5
    assert d_nocast > 1e-4
