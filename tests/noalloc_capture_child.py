"""Child process of tests/test_zz_no_alloc.py::test_noalloc_first_call_inside_graph_capture.

Runs in a fresh process so that the library's first call of
gllm_qkv_rope_kv_write_noalloc (which resolves the static scratch's device
address) happens inside a HIP graph capture.  Prints one line per step and
exits non-zero on a mismatch."""
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

import torch  # noqa: E402

from gllm_amd import _lib  # noqa: E402
from tests.test_zz_no_alloc import BF, DEV, _inputs  # noqa: E402


def main():
    lib = _lib.load()
    hidden, Hq, Hkv, D, n = 2048, 32, 8, 64, 64
    x, w, cos, sin, pos, slots, ns = _inputs(n, hidden, Hq, Hkv, D, 5)
    q_out = torch.full((n, Hq, D), 9.0, dtype=BF, device=DEV)
    kc = torch.full((ns, Hkv, D), 5.0, dtype=BF, device=DEV)
    vc = kc.clone()

    def args(q_o, k_c, v_c, xx, pp):
        return [xx.data_ptr(), hidden, xx.shape[0], hidden, w[0].data_ptr(), hidden, w[1].data_ptr(), hidden,
                w[2].data_ptr(), hidden, q_o.data_ptr(), Hq * D, 1, k_c.data_ptr(), v_c.data_ptr(), Hkv * D, ns,
                slots.data_ptr(), None, 0, cos.data_ptr(), sin.data_ptr(), pp.data_ptr(), D // 2, Hq, Hkv, D,
                _lib.DTYPE_BF16, _lib.DTYPE_BF16]

    # reference: the workspace entry point, eager
    need = lib.gllm_qkv_workspace_bytes(n, hidden, Hq, Hkv, D, 1)
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    rq, rk, rv = q_out.clone(), kc.clone(), vc.clone()
    _lib.check(lib.gllm_qkv_rope_kv_write(*args(rq, rk, rv, x, pos), ws.data_ptr(), need,
                                          _lib.stream_ptr(torch.device(DEV))))
    torch.cuda.synchronize()
    print("reference done", flush=True)
    # the first no-alloc call of the process, inside capture
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _lib.check(lib.gllm_qkv_rope_kv_write_noalloc(*args(q_out, kc, vc, x, pos),
                                                      _lib.stream_ptr(torch.device(DEV))))
    torch.cuda.synchronize()
    print("captured", flush=True)
    x2 = torch.randn(40, hidden, device=DEV).to(BF)
    for rep in range(3):
        q_out.fill_(9.0)
        kc.fill_(5.0)
        vc.fill_(5.0)
        # eager no-alloc call on other data between replays: the scratch then
        # holds another batch's partials, which the replay must overwrite
        oq, ok, ov = q_out.clone(), kc.clone(), vc.clone()
        _lib.check(lib.gllm_qkv_rope_kv_write_noalloc(*args(oq, ok, ov, x2, pos[:40]),
                                                      _lib.stream_ptr(torch.device(DEV))))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for a, b, nm in ((q_out, rq, "q"), (kc, rk, "k"), (vc, rv, "v")):
            if not torch.equal(a.view(torch.int16), b.view(torch.int16)):
                print(f"replay {rep}: {nm} differs", flush=True)
                return 1
        print(f"replay {rep} bit-exact", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
