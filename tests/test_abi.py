"""CPU checks of the C ABI: the library loads, exports every function the
header declares with a binding, and validates arguments without a GPU."""
import ctypes
import os
import re

import pytest

from gllm_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions():
    src = open(os.path.join(ROOT, "include", "gllm_attn.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(gllm_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = _header_functions()
    assert len(names) >= 10
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes binding"
    assert set(_lib.SIGNATURES) == set(names)
    assert lib.gllm_attn_version() == 1


def test_planner_host_logic():
    lib = _lib.load()
    h = ctypes.c_void_p()
    ql = (ctypes.c_int32 * 3)(1, 1, 40)
    sl = (ctypes.c_int32 * 3)(100, 2000, 80)
    assert lib.gllm_attn_plan_create(ctypes.byref(h), ql, sl, 3, 0, 32, 8, 64, 16, _lib.DTYPE_BF16, 128, 8) == 0
    info = (ctypes.c_int64 * 7)()
    assert lib.gllm_attn_plan_info(h, info, 7) == 0
    items, split, ndec, npf, parts, rows, hw = list(info)
    assert hw == 8
    # seq0: 1 split; seq1: 16 splits (one workgroup serves all 8 kv heads);
    # seq2 (40 rows x G=4 > 16): prefill, ceil(4 * 2 row tiles / 8) = 1 workgroup x 8 kv heads
    assert (items, split, ndec, npf, parts, rows) == (1 + 16 + 8, 128, 2, 1, 8 * 16, 42)
    assert lib.gllm_attn_plan_workspace_bytes(h) > 8 * 16 * 64 * 4
    info9 = (ctypes.c_int64 * 9)()
    assert lib.gllm_attn_plan_info(h, info9, 9) == 0
    assert info9[8] == 8                      # mixed launch: 8-wave prefill workgroups
    assert lib.gllm_attn_plan_destroy(h) == 0
    # prefill only: 100 rows x G=4 -> 4 row tiles x 4 heads = 16 waves -> 2 workgroups per kv head
    ql = (ctypes.c_int32 * 2)(100, 33)
    sl = (ctypes.c_int32 * 2)(100, 50)
    assert lib.gllm_attn_plan_create(ctypes.byref(h), ql, sl, 2, 0, 32, 8, 128, 16, _lib.DTYPE_BF16, 0, 0) == 0
    assert lib.gllm_attn_plan_info(h, info9, 9) == 0
    assert info9[8] == 8 and info9[2] == 0 and info9[3] == 2
    assert info9[0] == 8 * 2 + 8 * 1          # seq1: 2 row tiles x 4 heads = 8 waves -> 1 workgroup
    assert lib.gllm_attn_plan_destroy(h) == 0


def _plan_info(lib, ql, sl, hq, hkv, d, split=0, hw=0):
    h = ctypes.c_void_p()
    n = len(ql)
    rc = lib.gllm_attn_plan_create(ctypes.byref(h), (ctypes.c_int32 * n)(*ql), (ctypes.c_int32 * n)(*sl), n, 0,
                                   hq, hkv, d, 16, _lib.DTYPE_BF16, split, hw)
    if rc:
        return rc, None
    info = (ctypes.c_int64 * 10)()
    assert lib.gllm_attn_plan_info(h, info, 10) == 0
    assert lib.gllm_attn_plan_destroy(h) == 0
    return 0, dict(zip(("wgs", "split", "ndec", "npf", "parts", "rows", "hw", "dw", "pw", "segs"), list(info)))


def test_planner_page_balanced():
    """Page-balanced decode plans (GLLM_SPLIT_BALANCED = -1, or chosen for
    long-context batches): 16-key units per (sequence, kv-head group) dealt
    to min(units, resident slots) workgroups (256 CUs off-GPU: 512 at D = 64,
    256 at D = 128)."""
    from gllm_amd import workloads
    lib = _lib.load()
    # 7 + 125 units <= 512 workgroups: one unit each, every unit its own segment;
    # partials: 8 heads x segments of each split sequence
    rc, i = _plan_info(lib, [1, 1], [100, 2000], 32, 8, 64, split=-1)
    assert rc == 0 and (i["wgs"], i["segs"], i["parts"], i["hw"], i["split"]) == (132, 132, 8 * 132, 8, 0)
    # Hkv 12 -> 4 heads per workgroup, 3 groups; Hkv 2 -> 2
    assert _plan_info(lib, [1], [64], 48, 12, 64, split=-1)[1]["hw"] == 4
    assert _plan_info(lib, [1], [64], 16, 2, 64, split=-1)[1]["hw"] == 2
    # short contexts (config b) stay on the split planner, long ones (config e) go balanced
    b, e = workloads.config_b(), workloads.config_e()
    rc, i = _plan_info(lib, b.q_lens, b.seq_lens, 32, 8, 64)
    assert rc == 0 and i["segs"] == 0
    rc, i = _plan_info(lib, b.q_lens, b.seq_lens, 32, 8, 64, split=-1)
    assert rc == 0 and i["wgs"] == 512 and i["segs"] >= 512
    rc, i = _plan_info(lib, e.q_lens, e.seq_lens, 64, 8, 128)
    assert rc == 0 and i["wgs"] == 256 and i["segs"] >= 256 and i["hw"] == 8
    # a segment caches at most 512 block ids: >= 8192 keys per workgroup means cuts
    assert i["segs"] >= sum(-(-L // 8192) for L in e.seq_lens)
    # D = 128: the balanced plan needs >= 192 units (3072 keys) per workgroup,
    # so (d)'s 256 decodes (~137 units per workgroup) stay on the split planner
    d = workloads.config_d()
    rc, i = _plan_info(lib, d.q_lens[:256], d.seq_lens[:256], 32, 8, 128)
    assert rc == 0 and i["segs"] == 0 and i["split"] > 0
    rc, i = _plan_info(lib, [1] * 256, [191 * 16] * 256, 32, 8, 128)
    assert rc == 0 and i["segs"] == 0
    rc, i = _plan_info(lib, [1] * 256, [192 * 16] * 256, 32, 8, 128)
    assert rc == 0 and i["segs"] == 256 and i["wgs"] == 256
    # mixed batch, page-balanced on request: decode workgroups (a multiple of
    # 8, one per CU) plus one workgroup per prefill item; auto keeps the item plan
    rc, i = _plan_info(lib, d.q_lens, d.seq_lens, 32, 8, 128, split=-1)
    assert rc == 0 and i["npf"] == 4 and i["ndec"] == 256 and i["segs"] > 0
    kd = i["wgs"] - 4 * 8 * 8                       # 4 sequences x 8 kv heads x 8 items
    assert 0 < kd < 256 and kd % 8 == 0
    rc, i = _plan_info(lib, d.q_lens, d.seq_lens, 32, 8, 128)
    assert rc == 0 and i["segs"] == 0 and i["wgs"] == 4 * 8 * 8 + 256 * 8 // i["hw"]
    # a lone decode next to a prefill: one decode workgroup of one unit
    rc, i = _plan_info(lib, [1, 40], [10, 80], 32, 8, 64, split=-1)
    assert rc == 0 and (i["ndec"], i["npf"], i["segs"]) == (1, 1, 1)


@pytest.mark.parametrize("args,code", [
    (dict(ql=[0], sl=[5]), _lib.EINVAL),           # empty query
    (dict(ql=[6], sl=[5]), _lib.EINVAL),           # seq shorter than query
    (dict(hq=6, hkv=4), _lib.EINVAL),              # Hq not a multiple of Hkv
    (dict(bs=0), _lib.EINVAL),                     # block size < 1
    (dict(bs=65537), _lib.EINVAL),                 # block size above 65536
    (dict(d=97), _lib.EUNSUPPORTED),               # odd head_dim
    (dict(d=258), _lib.EUNSUPPORTED),              # head_dim above 256
    (dict(split=48), _lib.EINVAL),                 # split not a multiple of 32
    (dict(split=-2), _lib.EINVAL),                 # negative split other than GLLM_SPLIT_BALANCED
    (dict(hw=3), _lib.EINVAL),                     # heads per decode workgroup
])
def test_planner_rejects(args, code):
    lib = _lib.load()
    ql = args.get("ql", [1])
    sl = args.get("sl", [10])
    h = ctypes.c_void_p()
    rc = lib.gllm_attn_plan_create(ctypes.byref(h), (ctypes.c_int32 * 1)(*ql), (ctypes.c_int32 * 1)(*sl), 1, 0,
                                   args.get("hq", 8), args.get("hkv", 2), args.get("d", 64), args.get("bs", 16),
                                   _lib.DTYPE_BF16, args.get("split", 0), args.get("hw", 0))
    assert rc == code
    assert lib.gllm_attn_last_error()
    assert not h.value


def test_null_arguments_rejected():
    lib = _lib.load()
    rc = lib.gllm_paged_attention(None, None, 0, None, 0, None, None, 0, 0, None, 0, None, None, 0, 0, 1.0,
                                  _lib.DTYPE_BF16, _lib.DTYPE_BF16, None)
    assert rc == _lib.EINVAL
    rc = lib.gllm_attention_dense(None, 0, None, 0, 0, None, 0, 0, None, 0, 0, None, 0, 1, 1, 1, 1, 1, 64, 1.0,
                                  _lib.DTYPE_BF16, None)
    assert rc == _lib.EINVAL
    rc = lib.gllm_rope_kv_write(None, None, None, None, None, None, None, None, 0, None, None, None, 64, 1, 1, 1,
                                64, 64, 64, 64, 64, 64, 10, _lib.DTYPE_BF16, _lib.DTYPE_BF16, None)
    assert rc == _lib.EINVAL
