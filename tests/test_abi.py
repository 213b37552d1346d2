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


@pytest.mark.parametrize("args,code", [
    (dict(ql=[0], sl=[5]), _lib.EINVAL),           # empty query
    (dict(ql=[6], sl=[5]), _lib.EINVAL),           # seq shorter than query
    (dict(hq=6, hkv=4), _lib.EINVAL),              # Hq not a multiple of Hkv
    (dict(bs=12), _lib.EUNSUPPORTED),              # block size not a power of two
    (dict(d=96), _lib.EUNSUPPORTED),               # bf16 head_dim
    (dict(split=48), _lib.EINVAL),                 # split not a multiple of 32
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
