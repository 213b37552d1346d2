"""Fused QKV projection + RoPE + paged KV write (gllm/model/layers/attention.py:139-161)
against the oracle restatement.

The GEMM accumulates in fp32 in its own order, so a projected bf16 value may
differ from the correctly rounded one by one unit in the last place near a
rounding boundary (torch's own bf16 F.linear does the same); random-data
cases allow that on a small fraction of values.  With small-integer data
every dot product is exact in fp32 and bf16, so those cases pin the RoPE,
the casts and the slot writes bit for bit."""
import os

import pytest
import torch

from gllm_amd import paged
from oracle import projection as op
from oracle import rope as orope

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


def _inputs(n, hidden, Hq, Hkv, D, integer, seed, theta=500000.0, max_pos=4096):
    g = torch.Generator().manual_seed(seed)
    if integer:
        x = torch.randint(-1, 2, (n, hidden), generator=g).to(BF)
        w = [torch.randint(-1, 2, (h * D, hidden), generator=g).to(BF) for h in (Hq, Hkv, Hkv)]
    else:
        x = torch.randn(n, hidden, generator=g).to(BF)
        w = [(torch.randn(h * D, hidden, generator=g) / hidden ** 0.5).to(BF) for h in (Hq, Hkv, Hkv)]
    cos_t, sin_t = orope.rope_cache(max_pos, D, theta, BF)
    pos = torch.randint(0, max_pos, (n,), generator=g)
    num_slots = 2 * n + 16
    slots = torch.randperm(num_slots, generator=g)[:n].to(torch.int64)
    return x, w, cos_t, sin_t, pos, slots, num_slots


def _pair_norm(t):
    """|(x_d, x_{d+D/2})| per element: the rotation keeps it, so it bounds
    the error a one-ulp difference of the projected pair leaves after RoPE."""
    h = t.shape[-1] // 2
    r = (t[..., :h] ** 2 + t[..., h:] ** 2).sqrt()
    return torch.cat([r, r], -1)


def _close_bf16(got, want, what, rotated, frac=0.02):
    got, want = got.float().cpu(), want.float().cpu()
    diff = (got - want).abs()
    # a one-ulp difference of a projected value goes through RoPE's three
    # roundings: up to ~3 ulps of the pair's magnitude (4 allowed); v: 2 ulps
    if rotated:
        tol = torch.maximum(_pair_norm(got), _pair_norm(want)) * 2 ** -6 + 1e-6
    else:
        tol = torch.maximum(got.abs(), want.abs()) * 2 ** -7 + 1e-6
    assert bool((diff <= tol).all()), f"{what}: max diff {diff.max().item()} (worst ratio {(diff / tol).max().item():.2f})"
    assert (got != want).float().mean().item() <= frac, f"{what}: {(got != want).float().mean().item():.4f} differ"


def _run(n, hidden, Hq, Hkv, D, integer, seed, kv_dtype=BF, rotate_q=True, with_q=True, unfused_from=None):
    x, (wq, wk, wv), cos_t, sin_t, pos, slots, ns = _inputs(n, hidden, Hq, Hkv, D, integer, seed)
    sentinel = 3.0
    kc = torch.full((ns, Hkv, D), sentinel, dtype=BF).to(kv_dtype)
    vc = kc.clone()
    kc_ref, vc_ref = kc.clone(), vc.clone()
    q = paged.qkv_rope_kv_write(x.to(DEV), wq.to(DEV) if with_q else None, wk.to(DEV), wv.to(DEV),
                                cos_t.to(DEV), sin_t.to(DEV), kcg := kc.to(DEV), vcg := vc.to(DEV),
                                slots.to(DEV), rotate_q=rotate_q, rope_rows=pos.to(DEV), unfused_from=unfused_from)
    torch.cuda.synchronize()
    qr = op.qkv_rope_kv_write(x, wq, wk, wv, cos_t[pos], sin_t[pos], kc_ref, vc_ref, slots, Hkv, D)
    if not rotate_q:
        qr = op.linear(x, wq).view(n, Hq, D)
    return q, qr, kcg.cpu(), vcg.cpu(), kc_ref, vc_ref, slots, ns


@pytest.mark.parametrize("n,hidden,Hq,Hkv,D", [(1, 128, 4, 2, 64), (130, 128, 8, 2, 128), (300, 256, 16, 4, 64),
                                               (77, 96, 4, 4, 128),
                                               # prefill-sized batches, ragged last tile: 128-token
                                               # tiles, then 256-token x 2-head tiles in XCD order
                                               (2300, 128, 8, 2, 128), (6000, 64, 32, 8, 128)])
def test_qkv_exact_on_integer_data(n, hidden, Hq, Hkv, D):
    """Exact GEMM (small integers): q, the cached k (rotated) and v bit-exact,
    untouched slots keep their sentinel."""
    print(f"qkv exact n={n} hidden={hidden} Hq={Hq} Hkv={Hkv} D={D}", flush=True)
    q, qr, kc, vc, kr, vr, slots, ns = _run(n, hidden, Hq, Hkv, D, True, 11 + n)
    assert torch.equal(q.cpu().view(torch.int16), qr.view(torch.int16))
    assert torch.equal(kc.view(torch.int16), kr.view(torch.int16))
    assert torch.equal(vc.view(torch.int16), vr.view(torch.int16))


@pytest.mark.parametrize("n,hidden,Hq,Hkv,D", [(64, 2048, 32, 8, 64), (259, 4096, 32, 8, 128),
                                               (131, 1024, 8, 1, 128), (5, 512, 16, 16, 64),
                                               (2085, 1024, 8, 2, 128), (5500, 256, 32, 8, 128)])
def test_qkv_random_data(n, hidden, Hq, Hkv, D):
    """Llama-shaped projections (1B: hidden 2048 / D 64; 8B: 4096 / 128) on
    N(0,1) data: within the GEMM's accumulation-order rounding."""
    print(f"qkv random n={n} hidden={hidden} Hq={Hq} Hkv={Hkv} D={D}", flush=True)
    q, qr, kc, vc, kr, vr, slots, ns = _run(n, hidden, Hq, Hkv, D, False, 3 + n)
    _close_bf16(q, qr, "q", True)
    _close_bf16(kc[slots], kr[slots], "k", True)
    _close_bf16(vc[slots], vr[slots], "v", False)
    rest = torch.ones(ns, dtype=torch.bool)
    rest[slots] = False
    assert bool((kc[rest] == 3.0).all()) and bool((vc[rest] == 3.0).all())


def test_qkv_unrotated_q_and_fp8_cache():
    """rotate_q=False writes the plain projection (the attention kernels rotate
    q on load); an fp8 cache gets the rounded-like-torch cast of the bf16
    values (exact data, so byte-exact)."""
    print("qkv unrotated q, fp8 cache", flush=True)
    f8 = torch.float8_e4m3fn
    for n, hidden, Hq, Hkv, D in ((90, 128, 8, 2, 64), (6000, 64, 32, 8, 128)):   # small and large-batch tiles
        q, qr, kc, vc, kr, vr, slots, ns = _run(n, hidden, Hq, Hkv, D, True, 21, kv_dtype=f8, rotate_q=False)
        assert torch.equal(q.cpu().view(torch.int16), qr.view(torch.int16))
        assert torch.equal(kc.view(torch.uint8), kr.view(torch.uint8))
        assert torch.equal(vc.view(torch.uint8), vr.view(torch.uint8))


def test_qkv_without_q_and_padded_rows():
    """w_q=None skips the q heads; query_lens skips the reference's padded
    rows of a [B, T_q] layout (left in the cache as they were)."""
    print("qkv no q, padded rows", flush=True)
    B, Tq, hidden, Hkv, D = 3, 20, 128, 2, 128
    n = B * Tq
    x, (wq, wk, wv), cos_t, sin_t, pos, slots, ns = _inputs(n, hidden, 4, Hkv, D, True, 31)
    ql = torch.tensor([20, 7, 1], dtype=torch.int32)
    kc = torch.full((ns, Hkv, D), 3.0, dtype=BF)
    vc = kc.clone()
    kg, vg = kc.to(DEV), vc.to(DEV)
    out = paged.qkv_rope_kv_write(x.to(DEV), None, wk.to(DEV), wv.to(DEV), cos_t.to(DEV), sin_t.to(DEV), kg, vg,
                                  slots.to(DEV), query_lens=ql.to(DEV), rope_rows=pos.to(DEV))
    torch.cuda.synchronize()
    assert out is None
    real = (torch.arange(n) % Tq) < ql.repeat_interleave(Tq)
    op.qkv_rope_kv_write(x, None, wk, wv, cos_t[pos], sin_t[pos], kc, vc, slots, Hkv, D, real=real)
    assert torch.equal(kg.cpu().view(torch.int16), kc.view(torch.int16))
    assert torch.equal(vg.cpu().view(torch.int16), vc.view(torch.int16))


def test_qkv_rejects_bad_arguments():
    print("qkv errors", flush=True)
    x = torch.zeros(4, 100, dtype=BF, device=DEV)          # hidden not a multiple of 32
    w = torch.zeros(128, 100, dtype=BF, device=DEV)
    kc = torch.zeros(16, 1, 128, dtype=BF, device=DEV)
    cs = torch.zeros(4, 64, dtype=BF, device=DEV)
    sl = torch.arange(4, dtype=torch.int64, device=DEV)
    with pytest.raises(NotImplementedError):
        paged.qkv_rope_kv_write(x, None, w, w, cs, cs, kc, kc.clone(), sl)
    # the fused kernel projects in bf16 MFMA: its C entry point refuses other
    # model dtypes (the Python entry routes them to F.linear + the RoPE/KV
    # write kernel, test_qkv_other_model_dtypes_unfused_route)
    from gllm_amd import _lib
    lib = _lib.load()
    x32 = torch.zeros(4, 128, dtype=torch.float32, device=DEV)
    w32 = torch.zeros(128, 128, dtype=torch.float32, device=DEV)
    kc32, cs32 = kc.float(), cs.float()
    rc = lib.gllm_qkv_rope_kv_write(
        x32.data_ptr(), 128, 4, 128, None, 0, w32.data_ptr(), 128, w32.data_ptr(), 128, None, 0, 0,
        kc32.data_ptr(), kc32.clone().data_ptr(), 128, 16, sl.data_ptr(), None, 1, cs32.data_ptr(), cs32.data_ptr(),
        None, 64, 1, 1, 128, _lib.dtype_code(torch.float32), _lib.dtype_code(torch.float32), None, 0,
        _lib.stream_ptr(x32.device))
    assert rc == 2, rc                                   # GLLM_ATTN_EUNSUPPORTED


@pytest.mark.parametrize("dtype,kvd", [(torch.float32, torch.float32), (torch.float16, torch.float16),
                                       (torch.float32, torch.bfloat16)])
def test_qkv_other_model_dtypes_unfused_route(dtype, kvd):
    """fp32 and fp16 models (the reference takes any model dtype,
    model.py:64): the projections run as F.linear in the model dtype and
    the RoPE/KV write kernel rotates and stores.  Small integer data keep
    every product and sum exact, so q and the caches match the oracle bit
    for bit."""
    print(f"qkv unfused {dtype} kv={kvd}", flush=True)
    n, hidden, Hq, Hkv, D = 24, 512, 8, 2, 64
    x, w, cos_t, sin_t, pos, slots, num_slots = _inputs(n, hidden, Hq, Hkv, D, True, 77)
    x, w = x.to(dtype), [t.to(dtype) for t in w]
    cos_t, sin_t = orope.rope_cache(4096, D, 500000.0, dtype)
    kc_ref = torch.zeros(num_slots, Hkv, D, dtype=kvd)
    vc_ref = torch.zeros_like(kc_ref)
    qr = op.qkv_rope_kv_write(x, w[0], w[1], w[2], cos_t[pos], sin_t[pos], kc_ref, vc_ref, slots, Hkv, D)
    kc, vc = torch.zeros_like(kc_ref, device=DEV), torch.zeros_like(vc_ref, device=DEV)
    q = paged.qkv_rope_kv_write(x.to(DEV), w[0].to(DEV), w[1].to(DEV), w[2].to(DEV), cos_t.to(DEV), sin_t.to(DEV),
                                kc, vc, slots.to(DEV), rope_rows=pos.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(q.cpu(), qr)
    assert torch.equal(kc.cpu(), kc_ref) and torch.equal(vc.cpu(), vc_ref)


# hidden 544 (not a multiple of 64): the partial kernel's 32-wide K steps
@pytest.mark.parametrize("n,hidden,Hq,Hkv,D", [(64, 2048, 32, 8, 64), (70, 1024, 8, 2, 128), (100, 4096, 32, 8, 128),
                                               (40, 544, 4, 2, 64)])
def test_qkv_split_k_exact_and_matches_tile_path(n, hidden, Hq, Hkv, D):
    """Few tokens: the hidden dimension is split over workgroups (fp32
    partials summed in fixed order by a second launch).  Sparse small
    integers keep every partial and total exact, so q / K / V are bit-exact
    against the oracle and against the tile kernel (split_k=False)."""
    print(f"qkv split-k n={n} hidden={hidden} Hq={Hq} Hkv={Hkv} D={D}", flush=True)
    from gllm_amd import _lib
    lib = _lib.load()
    assert lib.gllm_qkv_workspace_bytes(n, hidden, Hq, Hkv, D, 1) > 0      # the split path is planned
    g = torch.Generator().manual_seed(40 + n)

    def sparse(*shape):
        v = torch.randint(-1, 2, shape, generator=g)
        return (v * (torch.rand(shape, generator=g) < 0.15)).to(BF)

    x = sparse(n, hidden)
    wq, wk, wv = sparse(Hq * D, hidden), sparse(Hkv * D, hidden), sparse(Hkv * D, hidden)
    cos_t, sin_t = orope.rope_cache(4096, D, 500000.0, BF)
    pos = torch.randint(0, 4096, (n,), generator=g)
    ns = 2 * n + 16
    slots = torch.randperm(ns, generator=g)[:n].to(torch.int64)
    outs = []
    for split in (True, False):
        kc = torch.full((ns, Hkv, D), 3.0, dtype=BF, device=DEV)
        vc = kc.clone()
        q = paged.qkv_rope_kv_write(x.to(DEV), wq.to(DEV), wk.to(DEV), wv.to(DEV), cos_t.to(DEV), sin_t.to(DEV),
                                    kc, vc, slots.to(DEV), rope_rows=pos.to(DEV), split_k=split, unfused_from=None)
        torch.cuda.synchronize()
        outs.append((q.cpu(), kc.cpu(), vc.cpu()))
    kr = torch.full((ns, Hkv, D), 3.0, dtype=BF)
    vr = kr.clone()
    qr = op.qkv_rope_kv_write(x, wq, wk, wv, cos_t[pos], sin_t[pos], kr, vr, slots, Hkv, D)
    for q, kc, vc in outs:
        assert torch.equal(q.view(torch.int16), qr.view(torch.int16))
        assert torch.equal(kc.view(torch.int16), kr.view(torch.int16))
        assert torch.equal(vc.view(torch.int16), vr.view(torch.int16))


def test_qkv_split_k_random_matches_tile_path():
    """N(0,1) data: split and tile paths differ only by the fp32 summation
    order of the projections (at most one bf16 ulp before RoPE)."""
    print("qkv split-k vs tile, random", flush=True)
    n, hidden, Hq, Hkv, D = 64, 2048, 32, 8, 64
    x, (wq, wk, wv), cos_t, sin_t, pos, slots, ns = _inputs(n, hidden, Hq, Hkv, D, False, 77)
    res = []
    for split in (True, False):
        kc = torch.zeros(ns, Hkv, D, dtype=BF, device=DEV)
        vc = torch.zeros_like(kc)
        q = paged.qkv_rope_kv_write(x.to(DEV), wq.to(DEV), wk.to(DEV), wv.to(DEV), cos_t.to(DEV), sin_t.to(DEV),
                                    kc, vc, slots.to(DEV), rope_rows=pos.to(DEV), split_k=split, unfused_from=None)
        torch.cuda.synchronize()
        res.append((q.cpu(), kc.cpu()[slots], vc.cpu()[slots]))
    _close_bf16(res[0][0], res[1][0], "q", True)
    _close_bf16(res[0][1], res[1][1], "k", True)
    _close_bf16(res[0][2], res[1][2], "v", False)


# (n, hidden, Hq, Hkv, D, kv dtype, rotate_q, with q): 1B / 8B head shapes
# (16-column and 32-column workgroups), a ragged second 16-token block, fp8
# cache, unrotated q, no q heads
SMALL_CASES = [(1, 2048, 32, 8, 64, BF, True, True), (32, 2048, 32, 8, 64, torch.float8_e4m3fn, True, True),
               (17, 4096, 32, 8, 128, BF, True, True), (9, 4096, 32, 8, 128, torch.float8_e4m3fn, False, True),
               (30, 768, 4, 4, 64, BF, True, False), (5, 256, 2, 1, 128, BF, False, True)]


@pytest.mark.parametrize("n,hidden,Hq,Hkv,D,kvd,rotate_q,with_q", SMALL_CASES)
def test_qkv_few_tokens_single_launch(n, hidden, Hq, Hkv, D, kvd, rotate_q, with_q):
    """Up to 32 tokens with hidden a multiple of 256 (<= 4096): one launch,
    each workgroup the whole hidden dimension of 16 or 32 output columns
    (eight waves split K and add their partials in LDS), so no workspace is
    planned.  Small-integer data: bit-exact against the oracle."""
    print(f"qkv few tokens n={n} hidden={hidden} Hq={Hq} Hkv={Hkv} D={D} kv={kvd} rot={rotate_q} q={with_q}",
          flush=True)
    from gllm_amd import _lib
    assert _lib.load().gllm_qkv_workspace_bytes(n, hidden, Hq, Hkv, D, int(with_q)) == 0
    q, qr, kc, vc, kr, vr, slots, ns = _run(n, hidden, Hq, Hkv, D, True, 50 + n, kv_dtype=kvd, rotate_q=rotate_q,
                                            with_q=with_q)
    if with_q:
        assert torch.equal(q.cpu().view(torch.int16), qr.view(torch.int16))
    else:
        assert q is None
    iv = torch.uint8 if kvd != BF else torch.int16
    assert torch.equal(kc.view(iv), kr.view(iv))
    assert torch.equal(vc.view(iv), vr.view(iv))


@pytest.mark.parametrize("n,hidden,Hq,Hkv,D", [(16, 4096, 32, 8, 128), (32, 2048, 32, 8, 64)])
def test_qkv_few_tokens_random_data(n, hidden, Hq, Hkv, D):
    """The single-launch path on N(0,1) data at the 8B / 1B shapes: within
    the GEMM's accumulation-order rounding of the oracle."""
    print(f"qkv few tokens random n={n} hidden={hidden} D={D}", flush=True)
    q, qr, kc, vc, kr, vr, slots, ns = _run(n, hidden, Hq, Hkv, D, False, 60 + n)
    _close_bf16(q, qr, "q", True)
    _close_bf16(kc[slots], kr[slots], "k", True)
    _close_bf16(vc[slots], vr[slots], "v", False)


def test_qkv_few_tokens_padded_rows():
    """Padded rows of a [B, T_q] layout on the single-launch path: skipped,
    their slots keep the sentinel."""
    print("qkv few tokens, padded rows", flush=True)
    B, Tq, hidden, Hq, Hkv, D = 4, 8, 512, 4, 2, 128
    n = B * Tq
    x, (wq, wk, wv), cos_t, sin_t, pos, slots, ns = _inputs(n, hidden, Hq, Hkv, D, True, 71)
    ql = torch.tensor([8, 3, 1, 5], dtype=torch.int32)
    kc = torch.full((ns, Hkv, D), 3.0, dtype=BF)
    vc = kc.clone()
    kg, vg = kc.to(DEV), vc.to(DEV)
    q = paged.qkv_rope_kv_write(x.to(DEV), wq.to(DEV), wk.to(DEV), wv.to(DEV), cos_t.to(DEV), sin_t.to(DEV), kg, vg,
                                slots.to(DEV), query_lens=ql.to(DEV), rope_rows=pos.to(DEV))
    torch.cuda.synchronize()
    real = (torch.arange(n) % Tq) < ql.repeat_interleave(Tq)
    qr = op.qkv_rope_kv_write(x, wq, wk, wv, cos_t[pos], sin_t[pos], kc, vc, slots, Hkv, D, real=real)
    assert torch.equal(kg.cpu().view(torch.int16), kc.view(torch.int16))
    assert torch.equal(vg.cpu().view(torch.int16), vc.view(torch.int16))
    assert torch.equal(q.cpu()[real].view(torch.int16), qr[real].view(torch.int16))


def _random_shapes(count, seed):
    """Seeded shapes over all three fused paths: up to 32 tokens (single
    launch), split-K (64- and 32-wide K steps) and the tile kernels."""
    import random
    r = random.Random(seed)
    out = []
    for _ in range(count):
        D = r.choice([64, 128])
        Hkv = r.choice([1, 2, 4])
        Hq = Hkv * r.choice([1, 2, 4])
        hidden = r.choice([32 * r.randint(8, 64), 256 * r.randint(1, 8)])   # 256 .. 2048; multiples of 32 / 256
        n = r.choice([r.randint(1, 32), r.randint(33, 160), r.randint(161, 700)])
        kvd = r.choice([BF, torch.float8_e4m3fn])
        out.append((n, hidden, Hq, Hkv, D, kvd, r.random() < 0.8, r.random() < 0.85))
    return out


# GLLM_QKV_RANDOM_SHAPES=n draws n seeded shapes instead of the default 16
@pytest.mark.parametrize("n,hidden,Hq,Hkv,D,kvd,rotate_q,with_q",
                         _random_shapes(int(os.environ.get("GLLM_QKV_RANDOM_SHAPES", "16")), 2024))
def test_qkv_random_shapes_exact(n, hidden, Hq, Hkv, D, kvd, rotate_q, with_q):
    """Random shapes (seeded), small-integer data: every fused path is
    bit-exact against the oracle."""
    print(f"qkv random shape n={n} hidden={hidden} Hq={Hq} Hkv={Hkv} D={D} kv={kvd} rot={rotate_q} q={with_q}",
          flush=True)
    q, qr, kc, vc, kr, vr, slots, ns = _run(n, hidden, Hq, Hkv, D, True, 90 + n, kv_dtype=kvd, rotate_q=rotate_q,
                                            with_q=with_q)
    if with_q:
        assert torch.equal(q.cpu().view(torch.int16), qr.view(torch.int16))
    iv = torch.uint8 if kvd != BF else torch.int16
    assert torch.equal(kc.view(iv), kr.view(iv))
    assert torch.equal(vc.view(iv), vr.view(iv))


@pytest.mark.parametrize("integer,rotate_q", [(True, True), (False, True), (True, False)])
def test_qkv_large_batch_unfused_route(integer, rotate_q):
    """From paged.QKV_UNFUSED_FROM tokens the projections go through F.linear
    (hipBLASLt) and then the RoPE + KV write kernel: same results as the
    oracle (exact on small-integer data, within the GEMM's rounding on N(0,1)
    data), untouched slots keep their sentinel."""
    n = paged.QKV_UNFUSED_FROM + 300
    print(f"qkv unfused route n={n} integer={integer} rotate_q={rotate_q}", flush=True)
    q, qr, kc, vc, kr, vr, slots, ns = _run(n, 256, 8, 2, 128, integer, 41, rotate_q=rotate_q,
                                            unfused_from=paged.QKV_UNFUSED_FROM)
    if integer:
        assert torch.equal(q.cpu().view(torch.int16), qr.view(torch.int16))
        assert torch.equal(kc.view(torch.int16), kr.view(torch.int16))
        assert torch.equal(vc.view(torch.int16), vr.view(torch.int16))
    else:
        _close_bf16(q, qr, "q", rotate_q)
        _close_bf16(kc[slots], kr[slots], "k", True)
        _close_bf16(vc[slots], vr[slots], "v", False)
    rest = torch.ones(ns, dtype=torch.bool)
    rest[slots] = False
    assert bool((kc[rest] == 3.0).all()) and bool((vc[rest] == 3.0).all())


@pytest.mark.parametrize("n,hidden,split_k", [(16, 256, True),      # one launch, <= 32 tokens
                                              (96, 1024, True),     # split-K partials + finish
                                              (600, 128, False)])   # tile kernel
@pytest.mark.parametrize("pad", ["q_out", "cache"])
def test_qkv_unaligned_row_strides(n, hidden, split_k, pad):
    """Row strides that are not multiples of 4 elements (q_out rows of
    Hq*D + 2, or cache slots of Hkv*D + 2) take the element-wise store path
    of every kernel: bit-exact against the oracle on exact data, and the
    padding elements between rows keep their sentinel."""
    print(f"qkv unaligned {pad} n={n} hidden={hidden} split_k={split_k}", flush=True)
    Hq, Hkv, D = 8, 2, 64
    x, (wq, wk, wv), cos_t, sin_t, pos, slots, ns = _inputs(n, hidden, Hq, Hkv, D, True, 50 + n)
    cpad = 2 if pad == "cache" else 0
    qpad = 2 if pad == "q_out" else 0
    kbuf = torch.full((ns, Hkv * D + cpad), 3.0, dtype=BF, device=DEV)
    vbuf = kbuf.clone()
    qbuf = torch.full((n, Hq * D + qpad), 7.0, dtype=BF, device=DEV)
    kc = kbuf[:, :Hkv * D].view(ns, Hkv, D)
    vc = vbuf[:, :Hkv * D].view(ns, Hkv, D)
    q_out = qbuf[:, :Hq * D].view(n, Hq, D)
    assert kc.stride(0) == Hkv * D + cpad and q_out.reshape(-1, Hq * D).stride(0) == Hq * D + qpad
    from gllm_amd import _lib
    wsb = _lib.load().gllm_qkv_workspace_bytes(n, hidden, Hq, Hkv, D, 1)
    assert (wsb > 0) == (split_k and n > 32)                  # the intended path is the one planned
    paged.qkv_rope_kv_write(x.to(DEV), wq.to(DEV), wk.to(DEV), wv.to(DEV), cos_t.to(DEV), sin_t.to(DEV), kc, vc,
                            slots.to(DEV), q_out=q_out, rope_rows=pos.to(DEV), split_k=split_k, unfused_from=None)
    torch.cuda.synchronize()
    kr = torch.full((ns, Hkv, D), 3.0, dtype=BF)
    vr = kr.clone()
    qr = op.qkv_rope_kv_write(x, wq, wk, wv, cos_t[pos], sin_t[pos], kr, vr, slots, Hkv, D)
    assert torch.equal(q_out.cpu().view(torch.int16), qr.view(torch.int16))
    assert torch.equal(kc.cpu().view(torch.int16), kr.view(torch.int16))
    assert torch.equal(vc.cpu().view(torch.int16), vr.view(torch.int16))
    assert bool((qbuf[:, Hq * D:] == 7.0).all()) and bool((kbuf[:, Hkv * D:] == 3.0).all())
    assert bool((vbuf[:, Hkv * D:] == 3.0).all())
