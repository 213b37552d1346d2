"""Python entry points over the C ABI: fused RoPE + KV write, batch plans and
paged attention.  Tensors are torch device tensors; every call is enqueued on
torch's current stream of the tensors' device.
"""
from __future__ import annotations

import ctypes
import math

import torch
import torch.nn.functional as F

from . import _lib


def _rows(t: torch.Tensor, heads: int, head_dim: int, name: str) -> int:
    """Row stride (elements) of a [..., heads, head_dim] tensor whose leading
    dims flatten to rows without a copy."""
    if t.dim() < 2 or t.shape[-1] != head_dim or t.shape[-2] != heads:
        raise ValueError(f"{name}: expected [..., {heads}, {head_dim}], got {tuple(t.shape)}")
    if t.stride(-1) != 1 or t.stride(-2) != head_dim:
        raise ValueError(f"{name}: head dim and heads must be contiguous")
    lead = t.shape[:-2]
    stride = t.stride(-3) if t.dim() >= 3 else heads * head_dim
    # leading dims must flatten to one row axis of constant stride
    expect = stride
    for d in range(t.dim() - 3, -1, -1):
        if t.shape[d] > 1 and t.stride(d) != expect:
            raise ValueError(f"{name}: leading dims do not flatten to rows")
        expect *= t.shape[d]
    del lead
    return stride


def rope_kv_write(k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                  k_cache: torch.Tensor, v_cache: torch.Tensor, slot_mapping: torch.Tensor,
                  query_lens: torch.Tensor | None = None, q: torch.Tensor | None = None,
                  q_out: torch.Tensor | None = None, rope_rows: torch.Tensor | None = None) -> None:
    """RoPE on k (and q -> q_out) plus the KV-cache write of
    ``gllm/model/layers/attention.py:151-161``.

    k/v ``[..., Hkv, D]`` (token rows), cos/sin ``[..., D/2]`` with one row per
    token (or ``rope_rows`` indexing a table), caches ``[num_slots, Hkv, D]``,
    ``slot_mapping`` int64 with one slot per token.  With ``query_lens``
    (padded ``[B, T_q]`` token layout) rows past each sequence's length are not
    written.
    """
    Hkv, D = k.shape[-2], k.shape[-1]
    if k.shape != v.shape:
        raise ValueError("k and v shapes differ")
    ks = _rows(k, Hkv, D, "k")
    vs = _rows(v, Hkv, D, "v")
    n = k.numel() // (Hkv * D)
    for t, nm in ((k_cache, "k_cache"), (v_cache, "v_cache")):
        if t.dim() != 3 or t.shape[1:] != (Hkv, D) or t.stride(2) != 1 or t.stride(1) != D:
            raise ValueError(f"{nm}: expected [num_slots, {Hkv}, {D}] with contiguous rows")
    if k_cache.stride(0) != v_cache.stride(0) or k_cache.shape[0] != v_cache.shape[0]:
        raise ValueError("k_cache and v_cache must have the same shape and slot stride")
    sm = slot_mapping.reshape(-1)
    if sm.dtype != torch.int64 or sm.numel() != n or not sm.is_contiguous():
        raise ValueError("slot_mapping must be contiguous int64 with one entry per token")
    cs = cos.reshape(-1, cos.shape[-1])
    sn = sin.reshape(-1, sin.shape[-1])
    if cs.stride(-1) != 1 or sn.stride(-1) != 1 or cs.stride(0) != sn.stride(0):
        raise ValueError("cos/sin must have contiguous rows of equal stride")
    if cs.dtype != k.dtype or sn.dtype != k.dtype:
        raise ValueError("cos/sin must be in the model dtype")
    if cs.shape[-1] < D // 2 or (rope_rows is None and cs.shape[0] < n):
        raise ValueError("cos/sin need one row of at least D/2 entries per token")
    tps = 0
    ql = None
    if query_lens is not None:
        ql = query_lens.to(torch.int32).contiguous()
        tps = n // ql.numel()
    qs = qos = 0
    Hq = 1
    if q_out is not None:
        Hq = q.shape[-2]
        qs = _rows(q, Hq, D, "q")
        qos = _rows(q_out, Hq, D, "q_out")
    rr = None
    if rope_rows is not None:
        rr = rope_rows.reshape(-1).to(torch.int64).contiguous()
    dev = k.device
    lib = _lib.load()
    _lib.check(lib.gllm_rope_kv_write(
        _lib.ptr(q), _lib.ptr(q_out), k.data_ptr(), v.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
        sm.data_ptr(), _lib.ptr(ql), tps, cs.data_ptr(), sn.data_ptr(), _lib.ptr(rr), cs.stride(0), n,
        Hq, Hkv, D, qs, ks, vs, qos, k_cache.stride(0), k_cache.shape[0],
        _lib.dtype_code(k.dtype), _lib.dtype_code(k_cache.dtype), _lib.stream_ptr(dev)))


# Token count from which qkv_rope_kv_write projects with hipBLASLt (three
# F.linear calls) and then runs the RoPE + KV write kernel: on MI355X the
# fused kernel is ahead up to ~2k tokens (8B shapes: 4.3x at 64 tokens, 1.1x
# at 2048) and behind from ~4k (0.90x at 4096, 0.82x at 19679 tokens).
QKV_UNFUSED_FROM = 3072


def qkv_rope_kv_write(x: torch.Tensor, w_q: torch.Tensor | None, w_k: torch.Tensor, w_v: torch.Tensor,
                      cos: torch.Tensor, sin: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                      slot_mapping: torch.Tensor, *, rotate_q: bool = True, q_out: torch.Tensor | None = None,
                      query_lens: torch.Tensor | None = None, rope_rows: torch.Tensor | None = None,
                      split_k: bool = True, unfused_from: int | None = QKV_UNFUSED_FROM):
    """Fused ``linear_q/k/v`` + RoPE + KV-cache write of
    ``gllm/model/layers/attention.py:139-161`` (bf16 model).

    x ``[..., hidden]`` token rows; weights as the checkpoint stores them
    (``w_q [Hq*D, hidden]``, ``w_k``/``w_v [Hkv*D, hidden]``, ``F.linear``
    convention); caches ``[num_slots, Hkv, D]``; cos/sin / ``rope_rows`` /
    ``query_lens`` / ``slot_mapping`` as in :func:`rope_kv_write`.  Returns q
    ``[N, Hq, D]`` (rotated if ``rotate_q``) or None when ``w_q`` is None.
    ``split_k``: let batches of few tokens split the hidden dimension over
    more workgroups (a cached device workspace); False forces the tile kernel.
    ``unfused_from``: from this many tokens the projections run as three
    ``F.linear`` (hipBLASLt) followed by :func:`rope_kv_write`, which is faster
    there; None runs the fused kernel at any size.  Head dims other than 64
    and 128, and models that are not bf16 (the fused kernel's projection is
    bf16 MFMA), always take the unfused path.
    """
    hidden = x.shape[-1]
    xs = x.reshape(-1, hidden)
    if xs.stride(-1) != 1:
        raise ValueError("x rows must be contiguous")
    n = xs.shape[0]
    for t, nm in ((k_cache, "k_cache"), (v_cache, "v_cache")):
        if t.dim() != 3 or t.stride(2) != 1 or t.stride(1) != t.shape[2]:
            raise ValueError(f"{nm}: expected [num_slots, Hkv, D] with contiguous rows")
    if k_cache.shape != v_cache.shape or k_cache.stride(0) != v_cache.stride(0):
        raise ValueError("k_cache and v_cache must have the same shape and slot stride")
    Hkv, D = k_cache.shape[1], k_cache.shape[2]
    for w, nm in ((w_k, "w_k"), (w_v, "w_v")) + (((w_q, "w_q"),) if w_q is not None else ()):
        if w.dim() != 2 or w.shape[1] != hidden or w.stride(1) != 1 or w.dtype != x.dtype:
            raise ValueError(f"{nm}: expected [heads * D, {hidden}] with contiguous rows in the model dtype")
    if w_k.shape[0] != Hkv * D or w_v.shape[0] != Hkv * D:
        raise ValueError("w_k / w_v must have num_kv_heads * head_dim rows")
    Hq = 0
    if w_q is not None:
        if w_q.shape[0] % D:
            raise ValueError("w_q rows must be a multiple of head_dim")
        Hq = w_q.shape[0] // D
        if q_out is None:
            q_out = torch.empty(n, Hq, D, dtype=x.dtype, device=x.device)
        if q_out.reshape(-1, Hq * D).shape[0] != n or q_out.stride(-1) != 1:
            raise ValueError("q_out must hold one contiguous row of Hq * D per token")
    sm = slot_mapping.reshape(-1)
    if sm.dtype != torch.int64 or sm.numel() != n or not sm.is_contiguous():
        raise ValueError("slot_mapping must be contiguous int64 with one entry per token")
    cs = cos.reshape(-1, cos.shape[-1])
    sn = sin.reshape(-1, sin.shape[-1])
    if cs.stride(-1) != 1 or sn.stride(-1) != 1 or cs.stride(0) != sn.stride(0):
        raise ValueError("cos/sin must have contiguous rows of equal stride")
    if cs.dtype != x.dtype or sn.dtype != x.dtype:
        raise ValueError("cos/sin must be in the model dtype")
    if cs.shape[-1] < D // 2 or (rope_rows is None and cs.shape[0] < n):
        raise ValueError("cos/sin need one row of at least D/2 entries per token")
    tps = 0
    ql = None
    if query_lens is not None:
        ql = query_lens.to(torch.int32).contiguous()
        tps = n // ql.numel()
    rr = None
    if rope_rows is not None:
        rr = rope_rows.reshape(-1).to(torch.int64).contiguous()
    if (unfused_from is not None and n >= unfused_from) or D not in (64, 128) or x.dtype != torch.bfloat16:
        k = F.linear(xs, w_k).view(n, Hkv, D)
        v = F.linear(xs, w_v).view(n, Hkv, D)
        q = F.linear(xs, w_q).view(n, Hq, D) if w_q is not None else None
        rotq = q is not None and rotate_q
        rope_kv_write(k, v, cos, sin, k_cache, v_cache, sm, query_lens=query_lens,
                      q=q if rotq else None, q_out=q_out.view(n, Hq, D) if rotq else None, rope_rows=rr)
        if q is not None and not rotate_q:
            q_out.view(n, Hq, D).copy_(q)
        return q_out
    lib = _lib.load()
    qrow = q_out.reshape(-1, Hq * D).stride(0) if q_out is not None else 0
    wsb = lib.gllm_qkv_workspace_bytes(n, hidden, max(Hq, 1), Hkv, D, int(w_q is not None)) if split_k else 0
    ws = _qkv_workspace(x.device, wsb) if wsb else None
    _lib.check(lib.gllm_qkv_rope_kv_write(
        xs.data_ptr(), xs.stride(0), n, hidden, _lib.ptr(w_q), w_q.stride(0) if w_q is not None else 0,
        w_k.data_ptr(), w_k.stride(0), w_v.data_ptr(), w_v.stride(0), _lib.ptr(q_out), qrow, int(bool(rotate_q)),
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.shape[0], sm.data_ptr(), _lib.ptr(ql),
        tps, cs.data_ptr(), sn.data_ptr(), _lib.ptr(rr), cs.stride(0), max(Hq, 1), Hkv, D,
        _lib.dtype_code(x.dtype), _lib.dtype_code(k_cache.dtype), _lib.ptr(ws), wsb, _lib.stream_ptr(x.device)))
    return q_out


_QKV_WS: dict = {}


def _qkv_workspace(device, nbytes: int) -> torch.Tensor:
    """Per-device scratch for the split-K projection (grown on demand, kept;
    fully rewritten by every call, so never cleared)."""
    key = torch.device(device)
    ws = _QKV_WS.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=key)
        _QKV_WS[key] = ws
    return ws


def rope_rotate(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                rope_rows: torch.Tensor | None = None) -> torch.Tensor:
    """Rotate-half RoPE of ``x [..., H, D]`` (``attention.py:91-118``),
    bit-identical to the reference's per-op rounding; returns a new tensor."""
    H, D = x.shape[-2], x.shape[-1]
    xs = _rows(x, H, D, "x")
    out = torch.empty_like(x, memory_format=torch.contiguous_format)
    n = x.numel() // (H * D)
    cs = cos.reshape(-1, cos.shape[-1])
    sn = sin.reshape(-1, sin.shape[-1])
    rr = None if rope_rows is None else rope_rows.reshape(-1).to(torch.int64).contiguous()
    if cs.shape[-1] < D // 2 or (rr is None and cs.shape[0] < n) or cs.stride(0) != sn.stride(0):
        raise ValueError("cos/sin need one row of at least D/2 entries per token")
    lib = _lib.load()
    _lib.check(lib.gllm_rope_kv_write(
        x.data_ptr(), out.data_ptr(), None, None, None, None, None, None, 0, cs.data_ptr(), sn.data_ptr(),
        _lib.ptr(rr), cs.stride(0), n, H, 1, D, xs, 0, 0, H * D, 0, 0,
        _lib.dtype_code(x.dtype), _lib.dtype_code(x.dtype), _lib.stream_ptr(x.device)))
    return out


def build_metadata(block_table: torch.Tensor, seq_lens: torch.Tensor, query_lens: torch.Tensor, block_size: int,
                   *, q_seq_stride: int = 0, num_rows: int | None = None):
    """Query-row slot mapping and positions on the device (``gllm/llm/llm.py:
    245-281`` without the per-row host loop or the dense bias).

    ``block_table`` int32 ``[B, W]`` (contiguous rows), ``seq_lens`` /
    ``query_lens`` int32 ``[B]`` on the same device.  ``q_seq_stride`` > 0:
    the reference's padded ``[B, T_q]`` rows (padded rows get slot 0);
    0: packed rows, and ``cu_seqlens`` (int32 ``[B+1]``) is returned too.
    ``num_rows`` (packed) is the total query rows; if omitted it is read back
    from the device (one synchronisation).  Returns
    ``(slot_mapping int64 [rows], positions int64 [rows], cu_seqlens or None)``.
    """
    B = int(seq_lens.shape[0])
    dev = block_table.device
    for t, nm in ((seq_lens, "seq_lens"), (query_lens, "query_lens"), (block_table, "block_table")):
        if t.dtype != torch.int32 or t.device != dev:
            raise ValueError(f"{nm} must be int32 on {dev}")
    if block_table.dim() != 2 or block_table.stride(1) != 1 or block_table.shape[0] < B or query_lens.shape[0] != B:
        raise ValueError("block_table must be [B, W] with contiguous rows and lengths [B]")
    if not seq_lens.is_contiguous() or not query_lens.is_contiguous():
        raise ValueError("lengths must be contiguous")
    if q_seq_stride > 0:
        rows = B * q_seq_stride
    else:
        rows = int(query_lens.sum().item()) if num_rows is None else int(num_rows)
    slots = torch.empty(rows, dtype=torch.int64, device=dev)
    pos = torch.empty(rows, dtype=torch.int64, device=dev)
    cu = torch.empty(B + 1, dtype=torch.int32, device=dev) if q_seq_stride == 0 else None
    lib = _lib.load()
    _lib.check(lib.gllm_build_metadata(block_table.data_ptr(), block_table.stride(0), block_table.shape[1],
                                       seq_lens.data_ptr(), query_lens.data_ptr(), B, q_seq_stride, block_size,
                                       slots.data_ptr(), pos.data_ptr(), _lib.ptr(cu), rows,
                                       _lib.stream_ptr(dev)))
    return slots, pos, cu


# split_tokens value that asks for a page-balanced decode plan (decode-only or mixed batches)
BALANCED = -1


class AttentionPlan:
    """Work plan for one batch (built once per engine step, reused by every
    layer).  Lengths are host ints, as ``gllm/llm/llm.py:233-241`` has them.

    ``q_seq_stride`` > 0: sequence i's rows start at ``i * q_seq_stride`` (the
    reference's padded ``[B, T_q]`` layout); 0: packed rows.  ``split_tokens``:
    0 lets the planner choose, a multiple of 32 fixes the decode split length,
    ``BALANCED`` deals the decode sequences' keys evenly to the workgroups (in
    a mixed batch: to part of the CUs, the prefill items run on the rest).
    """

    def __init__(self, query_lens, seq_lens, *, num_q_heads: int, num_kv_heads: int, head_dim: int,
                 block_size: int, dtype: torch.dtype, device, q_seq_stride: int = 0,
                 split_tokens: int = 0, heads_per_wg: int = 0):
        ql = [int(x) for x in query_lens]
        sl = [int(x) for x in seq_lens]
        if len(ql) != len(sl):
            raise ValueError("query_lens and seq_lens differ in length")
        lib = _lib.load()
        self._lib = lib
        self._h = ctypes.c_void_p()
        qa = (ctypes.c_int32 * max(len(ql), 1))(*ql)
        sa = (ctypes.c_int32 * max(len(sl), 1))(*sl)
        _lib.check(lib.gllm_attn_plan_create(ctypes.byref(self._h), qa, sa, len(ql), q_seq_stride,
                                             num_q_heads, num_kv_heads, head_dim, block_size,
                                             _lib.dtype_code(dtype), split_tokens, heads_per_wg))
        self.num_q_heads, self.num_kv_heads, self.head_dim = num_q_heads, num_kv_heads, head_dim
        self.block_size, self.dtype = block_size, dtype
        self.query_lens, self.seq_lens = ql, sl
        self.q_seq_stride = q_seq_stride
        self.device = torch.device(device)
        nbytes = lib.gllm_attn_plan_workspace_bytes(self._h)
        self.workspace = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        _lib.check(lib.gllm_attn_plan_upload(self._h, self.workspace.data_ptr(), nbytes,
                                             _lib.stream_ptr(self.device)))
        arr = (ctypes.c_int64 * 10)()
        _lib.check(lib.gllm_attn_plan_info(self._h, arr, 10))
        keys = ("work_items", "split_tokens", "decode_seqs", "prefill_seqs", "partials", "rows", "heads_per_wg",
                "decode_waves", "prefill_waves", "decode_segments")
        self._info = dict(zip(keys, list(arr)))
        # facts every launch checks, computed once (a plan serves every layer of a step)
        self.rows = self._info["rows"]
        self.max_seq_len = max(sl, default=0)
        self.table_width = -(-self.max_seq_len // block_size)

    @property
    def info(self) -> dict:
        return dict(self._info)

    def __del__(self):
        h = getattr(self, "_h", None)
        lib = getattr(self, "_lib", None)
        if h is not None and h.value and lib is not None:
            try:
                lib.gllm_attn_plan_destroy(h)
            except Exception:      # interpreter shutdown: ctypes may already be torn down
                return
            self._h = None


def fused_kv_write_ok(plan: AttentionPlan, kv_dtype: torch.dtype) -> bool:
    """Whether :func:`paged_attention` can take ``kv_new`` for this plan and
    cache dtype: every sequence on the decode path of the kernel that runs
    (MFMA kernels: query_len x G <= 16; generic kernel: query_len <= 16)."""
    if not plan.query_lens:
        return False
    mfma = (plan.dtype in (torch.bfloat16, torch.float16) and plan.head_dim in (64, 128)
            and kv_dtype in (plan.dtype, torch.float8_e4m3fn))
    G = plan.num_q_heads // plan.num_kv_heads
    if mfma:
        return max(plan.query_lens) * G <= 16
    return max(plan.query_lens) <= 16


def paged_attention(plan: AttentionPlan, q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                    block_table: torch.Tensor, out: torch.Tensor | None = None,
                    rope: tuple | None = None, scale: float | None = None,
                    kv_new: tuple | None = None) -> torch.Tensor:
    """Attention over the paged cache for every query row in ``plan``.

    q ``[rows, Hq, D]`` or ``[B, T_q, Hq, D]`` (rows flattened), caches
    ``[num_slots, Hkv, D]``, block_table int32 ``[B, W]``.  ``rope`` =
    ``(cos, sin, mode)`` with mode ``"position"`` (table rows ``c_i + r``) or
    ``"row"`` (one cos/sin row per query row, the reference's gathered
    ``cos_pos``) rotates q on load.  ``kv_new`` = ``(k, v)``, one row per
    query row in q's layout (``[..., Hkv, D]``): the new tokens' K/V, rotated
    (k) and written into the cache at their keys' slots by the same launch
    (``attention.py:151-161`` + this attention; the plan must pass
    :func:`fused_kv_write_ok`).  Returns ``out`` (same layout as q).
    """
    Hq, Hkv, D = plan.num_q_heads, plan.num_kv_heads, plan.head_dim
    qs = _rows(q, Hq, D, "q")
    if out is None:
        out = torch.empty_like(q, memory_format=torch.contiguous_format)
    os_ = _rows(out, Hq, D, "out")
    if q.dtype != plan.dtype or out.dtype != plan.dtype:
        raise ValueError("q/out dtype differs from the plan's")
    for t, nm in ((k_cache, "k_cache"), (v_cache, "v_cache")):
        if t.dim() != 3 or t.shape[1:] != (Hkv, D) or t.stride(2) != 1 or t.stride(1) != D:
            raise ValueError(f"{nm}: expected [num_slots, {Hkv}, {D}] with contiguous rows")
    if k_cache.stride(0) != v_cache.stride(0):
        raise ValueError("k_cache and v_cache slot strides differ")
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.stride(1) != 1:
        raise ValueError("block_table must be int32 [B, W] with contiguous rows")
    if block_table.shape[0] < len(plan.query_lens):
        raise ValueError("block_table has fewer rows than the plan's sequences")
    if block_table.shape[1] < plan.table_width:
        raise ValueError(f"block_table width {block_table.shape[1]} < {plan.table_width} blocks the longest "
                         "sequence needs")
    rows = q.numel() // (Hq * D)
    if rows < plan.rows:
        raise ValueError(f"q has {rows} rows, the plan addresses {plan.rows}")
    cos_p = sin_p = None
    rs = 0
    mode = _lib.ROPE_NONE
    if rope is not None:
        cos, sin, m = rope
        mode = {"position": _lib.ROPE_BY_POSITION, "row": _lib.ROPE_BY_ROW}[m]
        cos = cos.reshape(-1, cos.shape[-1])
        sin = sin.reshape(-1, sin.shape[-1])
        if cos.stride(-1) != 1 or sin.stride(-1) != 1 or cos.stride(0) != sin.stride(0):
            raise ValueError("cos/sin must have contiguous rows of equal stride")
        if cos.dtype != q.dtype:
            raise ValueError("cos/sin must be in the model dtype")
        need_rows = plan.max_seq_len if m == "position" else plan.rows
        if cos.shape[0] < need_rows or cos.shape[1] < D // 2:
            raise ValueError(f"cos/sin have {cos.shape[0]} rows, {need_rows} needed")
        cos_p, sin_p, rs = cos.data_ptr(), sin.data_ptr(), cos.stride(0)
    sc = 1.0 / math.sqrt(D) if scale is None else float(scale)
    num_blocks = k_cache.shape[0] // plan.block_size
    lib = _lib.load()
    if kv_new is not None:
        kn, vn = kv_new
        if kn.dtype != q.dtype or vn.dtype != q.dtype:
            raise ValueError("k_new / v_new must be in the model dtype")
        ks = _rows(kn, Hkv, D, "k_new")
        vs = _rows(vn, Hkv, D, "v_new")
        if kn.numel() // (Hkv * D) < plan.rows or vn.numel() // (Hkv * D) < plan.rows:
            raise ValueError("k_new / v_new need one row per query row of the plan")
        _lib.check(lib.gllm_paged_attention_write_kv(
            plan._h, q.data_ptr(), qs, out.data_ptr(), os_, k_cache.data_ptr(), v_cache.data_ptr(),
            k_cache.stride(0), num_blocks, block_table.data_ptr(), block_table.stride(0), kn.data_ptr(), ks,
            vn.data_ptr(), vs, cos_p, sin_p, rs, mode, sc, _lib.dtype_code(q.dtype), _lib.dtype_code(k_cache.dtype),
            _lib.stream_ptr(q.device)))
        return out
    _lib.check(lib.gllm_paged_attention(
        plan._h, q.data_ptr(), qs, out.data_ptr(), os_, k_cache.data_ptr(), v_cache.data_ptr(),
        k_cache.stride(0), num_blocks, block_table.data_ptr(), block_table.stride(0), cos_p, sin_p, rs, mode,
        sc, _lib.dtype_code(q.dtype), _lib.dtype_code(k_cache.dtype), _lib.stream_ptr(q.device)))
    return out
