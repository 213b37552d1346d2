"""ctypes binding of libgllm_attn.so (declared in include/gllm_attn.h).

The library is built in-tree by ``gllm_amd.build``.  There is no fallback:
if the shared object is missing or fails to load, every op raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libgllm_attn.so")

OK, EINVAL, EUNSUPPORTED, EHIP = 0, 1, 2, 3
DTYPE_F32, DTYPE_BF16, DTYPE_FP8_E4M3, DTYPE_F16 = 0, 1, 2, 3
ROPE_NONE, ROPE_BY_POSITION, ROPE_BY_ROW = 0, 1, 2

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/gllm_attn.h
SIGNATURES = {
    "gllm_attn_last_error": (ctypes.c_char_p, []),
    "gllm_attn_version": (ctypes.c_int, []),
    "gllm_rope_kv_write": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _p, _p, _i64, _i64,
                                          _i32, _i32, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _p]),
    "gllm_attn_plan_create": (ctypes.c_int, [ctypes.POINTER(_p), _p, _p, _i32, _i64, _i32, _i32, _i32,
                                             _i32, _i32, _i32, _i32]),
    "gllm_attn_plan_workspace_bytes": (_sz, [_p]),
    "gllm_attn_plan_upload": (ctypes.c_int, [_p, _p, _sz, _p]),
    "gllm_attn_plan_info": (ctypes.c_int, [_p, ctypes.POINTER(_i64), _i32]),
    "gllm_attn_plan_destroy": (ctypes.c_int, [_p]),
    "gllm_paged_attention": (ctypes.c_int, [_p, _p, _i64, _p, _i64, _p, _p, _i64, _i64, _p, _i64, _p, _p,
                                            _i64, _i32, _f32, _i32, _i32, _p]),
    "gllm_paged_attention_write_kv": (ctypes.c_int, [_p, _p, _i64, _p, _i64, _p, _p, _i64, _i64, _p, _i64, _p, _i64,
                                                     _p, _i64, _p, _p, _i64, _i32, _f32, _i32, _i32, _p]),
    "gllm_build_metadata": (ctypes.c_int, [_p, _i64, _i64, _p, _p, _i32, _i64, _i32, _p, _p, _p, _i64, _p]),
    "gllm_qkv_rope_kv_write": (ctypes.c_int, [_p, _i64, _i64, _i32, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _i32,
                                              _p, _p, _i64, _i64, _p, _p, _i64, _p, _p, _p, _i64, _i32, _i32, _i32,
                                              _i32, _i32, _p, _sz, _p]),
    "gllm_qkv_rope_kv_write_noalloc": (ctypes.c_int, [_p, _i64, _i64, _i32, _p, _i64, _p, _i64, _p, _i64, _p, _i64,
                                                      _i32, _p, _p, _i64, _i64, _p, _p, _i64, _p, _p, _p, _i64, _i32,
                                                      _i32, _i32, _i32, _i32, _p]),
    "gllm_qkv_workspace_bytes": (_sz, [_i64, _i32, _i32, _i32, _i32, _i32]),
    "gllm_attention_dense": (ctypes.c_int, [_p, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p,
                                            _i64, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _p]),
}

_lock = threading.Lock()
_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load (once) and return the library; raises if it is not built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise RuntimeError(
                f"libgllm_attn.so not found at {path}; build it with `python -m gllm_amd.build` "
                "(there is no CPU fallback)")
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def check(rc: int) -> None:
    if rc == OK:
        return
    msg = load().gllm_attn_last_error().decode()
    if rc == EINVAL:
        raise ValueError(msg)
    if rc == EUNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return DTYPE_BF16
    if dt == torch.float32:
        return DTYPE_F32
    if dt == torch.float16:
        return DTYPE_F16
    if dt == torch.float8_e4m3fn:
        return DTYPE_FP8_E4M3
    raise NotImplementedError(f"dtype {dt} is not supported (float32, bfloat16, float16; float8_e4m3fn for the "
                              "KV cache)")


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()
