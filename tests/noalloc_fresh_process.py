"""Fresh-process checks of gdn_prefill_launch_noalloc, run by tests/test_zz_no_alloc.py in
a child process (one at a time), because they need a process in which no noalloc call has
happened yet. Prints one JSON line.

1. Device memory: free bytes after a decode and a workspace prefill, then after the first
   noalloc call (the static scratch is taken only then).
2. A first noalloc call inside a stream capture fails cleanly (GDN_EINVAL, nothing
   recorded); after an eager call, a captured noalloc prefill replays bit-identically to
   the eager result, three times, with other noalloc calls between the replays.
"""
import ctypes
import json
import os
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (REPO, os.path.join(REPO, "mlsys26-flashinfer-ai-kernel-generation-contest_amd")):
    sys.path.insert(0, p)

import torch  # noqa: E402

from gdn_hip import _lib, gdn_decode, gdn_prefill  # noqa: E402
from gdn_hip.api import _prefill_marshal  # noqa: E402
from gdn_hip.inputs import decode_inputs, prefill_inputs  # noqa: E402


def noalloc(lib, g, out, ns):
    P, _, _, copy_back, keep, stream = _prefill_marshal(*g.args(), out, ns,
                                                        with_workspace=False)
    assert not copy_back
    rc = lib.gdn_prefill_launch_noalloc(ctypes.byref(P), ctypes.c_void_p(stream.cuda_stream))
    return rc, _lib.last_error(), keep


def main():
    dev = torch.device("cuda", 0)
    lib = _lib.load()
    res = {}
    d = decode_inputs(4, seed=1).to(dev)
    gdn_decode(*d.args())
    p = prefill_inputs([300, 77], seed=2, with_state=True).to(dev)
    gdn_prefill(*p.args())
    torch.cuda.synchronize()
    res["free_before"] = torch.cuda.mem_get_info(dev)[0]
    T, N = p.q.shape[0], 2
    out = torch.empty((T, 32, 128), dtype=torch.bfloat16, device=dev)
    ns = torch.empty((N, 32, 128, 128), dtype=torch.float32, device=dev)
    # (1) first call inside a capture: refused before anything is recorded
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc, msg, keep = noalloc(lib, p, out, ns)
    res["first_in_capture_rc"], res["first_in_capture_msg"] = rc, msg
    torch.cuda.synchronize()
    res["free_after_refused"] = torch.cuda.mem_get_info(dev)[0]
    # (2) eager first call, then a capture
    rc, msg, keep = noalloc(lib, p, out, ns)
    torch.cuda.synchronize()
    res["eager_rc"] = rc
    res["free_after_first_call"] = torch.cuda.mem_get_info(dev)[0]
    eo, en = out.clone(), ns.clone()
    out.fill_(7.0)
    ns.fill_(7.0)
    torch.cuda.synchronize()
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2):
        rc2, _, keep2 = noalloc(lib, p, out, ns)
    res["capture_rc"] = rc2
    other = prefill_inputs([1000, 64, 3], seed=9, with_state=False).to(dev)
    oo = torch.empty((other.q.shape[0], 32, 128), dtype=torch.bfloat16, device=dev)
    on = torch.empty((3, 32, 128, 128), dtype=torch.float32, device=dev)
    same = []
    for _ in range(3):
        out.fill_(7.0)
        ns.fill_(7.0)
        torch.cuda.synchronize()
        g2.replay()
        torch.cuda.synchronize()
        same.append(bool(torch.equal(out, eo) and torch.equal(ns, en)))
        noalloc(lib, other, oo, on)  # another call rewrites the shared scratch
        torch.cuda.synchronize()
    res["replays_bitwise"] = same
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
