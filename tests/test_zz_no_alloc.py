"""gllm_qkv_rope_kv_write_noalloc (static scratch, no allocation) against
gllm_qkv_rope_kv_write with a caller workspace: bit-identical q, K and V on
two calls in a row, the second with fewer tokens (the scratch keeps the
first call's partials), plus the size limit's error."""
import ctypes

import pytest
import torch

from gllm_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


def _inputs(n, hidden, Hq, Hkv, D, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, hidden, generator=g).to(BF).to(DEV)
    w = [(torch.randn(h * D, hidden, generator=g) / hidden ** 0.5).to(BF).to(DEV) for h in (Hq, Hkv, Hkv)]
    ang = torch.arange(4096).unsqueeze(1) * 500000.0 ** (-2 * torch.arange(D // 2) / D)
    cos, sin = torch.cos(ang).to(BF).to(DEV), torch.sin(ang).to(BF).to(DEV)
    pos = torch.randint(0, 4096, (n,), generator=g).to(DEV)
    ns = n + 64
    slots = torch.randperm(ns, generator=g)[:n].to(DEV)
    return x, w, cos, sin, pos, slots, ns


def _call(lib, noalloc, x, w, cos, sin, pos, slots, ns, Hq, Hkv, D, ws=None):
    n, hidden = x.shape
    q_out = torch.full((n, Hq, D), 9.0, dtype=BF, device=DEV)
    kc = torch.full((ns, Hkv, D), 5.0, dtype=BF, device=DEV)
    vc = kc.clone()
    args = [x.data_ptr(), hidden, n, hidden, w[0].data_ptr(), hidden, w[1].data_ptr(), hidden, w[2].data_ptr(),
            hidden, q_out.data_ptr(), Hq * D, 1, kc.data_ptr(), vc.data_ptr(), Hkv * D, ns, slots.data_ptr(), None, 0,
            cos.data_ptr(), sin.data_ptr(), pos.data_ptr(), D // 2, Hq, Hkv, D, _lib.DTYPE_BF16, _lib.DTYPE_BF16]
    if noalloc:
        rc = lib.gllm_qkv_rope_kv_write_noalloc(*args, _lib.stream_ptr(torch.device(DEV)))
    else:
        rc = lib.gllm_qkv_rope_kv_write(*args, _lib.ptr(ws), 0 if ws is None else ws.numel(),
                                        _lib.stream_ptr(torch.device(DEV)))
    _lib.check(rc)
    torch.cuda.synchronize()
    return q_out.cpu(), kc.cpu(), vc.cpu()


@pytest.mark.parametrize("hidden,Hq,Hkv,D", [(2048, 32, 8, 64), (4096, 32, 8, 128)])
def test_noalloc_matches_workspace_entry_point(hidden, Hq, Hkv, D):
    print(f"qkv noalloc hidden={hidden} D={D}", flush=True)
    lib = _lib.load()
    for n, seed in ((64, 1), (40, 2)):            # second call smaller: stale partials must not leak
        inp = _inputs(n, hidden, Hq, Hkv, D, seed)
        need = lib.gllm_qkv_workspace_bytes(n, hidden, Hq, Hkv, D, 1)
        assert need > 0                           # the split-K path (the one with scratch) runs
        ws = torch.empty(need, dtype=torch.uint8, device=DEV)
        ref = _call(lib, False, *inp, Hq, Hkv, D, ws=ws)
        got = _call(lib, True, *inp, Hq, Hkv, D)
        for a, b in zip(got, ref):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_noalloc_rejects_partials_beyond_the_scratch():
    """A batch whose split-K partials exceed the 24 MiB scratch is refused
    with a clear error (buffers are real and sized, so nothing would read out
    of bounds even if it were not)."""
    lib = _lib.load()
    hidden, Hkv, D = 512, 1, 128
    cand = None
    for heads in range(40, 256, 7):
        for n in (128, 192, 256, 384, 512):
            if lib.gllm_qkv_workspace_bytes(n, hidden, heads, Hkv, D, 1) > (24 << 20):
                cand = (heads, n)
                break
        if cand:
            break
    if cand is None:
        pytest.skip("no batch on this GPU needs more than the static scratch")
    Hq, n = cand
    print(f"qkv noalloc limit Hq={Hq} n={n}", flush=True)
    inp = _inputs(n, hidden, Hq, Hkv, D, 3)
    with pytest.raises(NotImplementedError, match="static scratch"):
        _call(lib, True, *inp, Hq, Hkv, D)


def test_noalloc_first_call_inside_graph_capture():
    """The use case of the no-alloc entry point: a caller under HIP graph
    capture.  In a fresh process (so the scratch address is resolved by a
    call made inside capture), the captured call replays bit-exact against
    the workspace entry point three times, with eager no-alloc calls on
    other data between the replays."""
    import os
    import subprocess
    import sys
    here = os.path.dirname(os.path.abspath(__file__))
    print("qkv noalloc: first call inside graph capture (child process)", flush=True)
    r = subprocess.run([sys.executable, "-u", os.path.join(here, "noalloc_capture_child.py")],
                       capture_output=True, text=True, timeout=110)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, r.stdout[-500:] + r.stderr[-1500:]
    assert r.stdout.count("bit-exact") == 3
