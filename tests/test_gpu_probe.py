"""The box-ceiling probes of bench.py (libgllm_probe.so) run at small sizes
and return sane figures: the read stream and the L2 -> LDS copies complete,
8 bf16 32x32x16 MFMAs take at least 8 x 32 cycles, interleaved FMAs cost
extra, and an empty grid launches."""
import ctypes

import pytest
import torch

from gllm_amd import _lib
from gllm_amd import build as gb

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _lib_probe():
    lib = ctypes.CDLL(gb.PROBE_LIB)
    p, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    lib.gllm_probe_read.argtypes = [p, i64, i32, p, p]
    lib.gllm_probe_lds_dma.argtypes = [p, i64, i32, i32, p, p]
    lib.gllm_probe_mfma.argtypes = [i32, i32, p, p]
    lib.gllm_probe_empty.argtypes = [i32, i32, i32, p, p]
    return lib


def test_probes_run():
    print("probes", flush=True)
    lib = _lib_probe()
    dev = torch.device(DEV, 0)
    st = _lib.stream_ptr(dev)
    sink = torch.zeros(64, dtype=torch.int32, device=dev)
    buf = torch.ones(16 * 32768, dtype=torch.uint8, device=dev)          # 16 workgroups x 32 KB
    assert lib.gllm_probe_read(buf.data_ptr(), buf.numel(), 16, sink.data_ptr(), st) == 0
    win = torch.ones(1 << 16, dtype=torch.uint8, device=dev)
    assert lib.gllm_probe_lds_dma(win.data_ptr(), win.numel(), 16, 64, sink.data_ptr(), st) == 0
    mf = torch.zeros(2, 4, dtype=torch.int64, device=dev)
    for mode in (0, 1):
        assert lib.gllm_probe_mfma(mode, 64, mf[mode].data_ptr(), st) == 0
    assert lib.gllm_probe_empty(64, 256, 4096, sink.data_ptr(), st) == 0
    torch.cuda.synchronize()
    m = mf.cpu()
    assert m[0, 0] >= 8 * 32 and m[0, 3] == 64 and m[0, 1] > 0
    assert m[1, 0] > m[0, 0]
