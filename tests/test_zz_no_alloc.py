"""gdn_prefill_launch_noalloc (static device scratch, no allocation) against
gdn_prefill_launch (caller-owned workspace), both called through the C ABI on the same
inputs: bit-identical outputs and states on two calls in a row, the second smaller than
the first, and a clear rejection of a size beyond the static scratch. Under HIP graph
capture: replays match the eager call, and (in a fresh child process) a first call inside
a capture is refused cleanly; the same child measures when the scratch is taken."""
import ctypes
import json
import os
import subprocess
import sys

import pytest
import torch

from gdn_hip import _lib
from gdn_hip.api import _prefill_marshal
from gdn_hip.inputs import prefill_inputs, varlen_lengths
from gdn_hip.parity import check_output, check_state
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu


def _both(dev, lens, seed, with_state):
    inp = prefill_inputs(lens, seed=seed, with_state=with_state)
    g = inp.to(dev)
    T, N = g.q.shape[0], len(lens)
    outs = []
    lib = _lib.load()
    for noalloc in (False, True):
        out = torch.full((T, 32, 128), 5.0, dtype=torch.bfloat16, device=dev)
        ns = torch.full((N, 32, 128, 128), 5.0, dtype=torch.float32, device=dev)
        P, _, _, copy_back, keep, stream = _prefill_marshal(
            *g.args(), out, ns, with_workspace=not noalloc)
        assert not copy_back
        fn = lib.gdn_prefill_launch_noalloc if noalloc else lib.gdn_prefill_launch
        print(f"[noalloc={noalloc}] T={T} N={N} launching", flush=True)
        _lib.check(fn(ctypes.byref(P), ctypes.c_void_p(stream.cuda_stream)), fn.__name__)
        torch.cuda.synchronize()
        outs.append((out, ns))
        del keep
    (o1, s1), (o2, s2) = outs
    print(f"[noalloc] lens={lens[:6]}... bitwise output {torch.equal(o1, o2)} "
          f"state {torch.equal(s1, s2)}", flush=True)
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
    return inp, o2, s2


def test_noalloc_matches_workspace_entry_point(dev):
    lib = _lib.load()
    cap = lib.gdn_prefill_noalloc_capacity()
    big = varlen_lengths(16, seed=0)  # the 8172-token workload
    need = lib.gdn_prefill_workspace_size(sum(big), len(big), 16, 32, 128)
    assert 0 < need <= cap
    _both(dev, big, 0, True)
    # second call smaller, after the first left its tables in the shared scratch
    inp, o, s = _both(dev, [300, 5, 129], 7, False)
    ref_o, ref_s = O.prefill(*inp.args())
    vo, vs = check_output(o, ref_o), check_state(s, ref_s)
    print(f"[noalloc small] output {vo} | state {vs}", flush=True)
    assert vo.ok and vs.ok


def test_noalloc_rejects_oversize(dev):
    lib = _lib.load()
    cap = lib.gdn_prefill_noalloc_capacity()
    T = 65536
    assert lib.gdn_prefill_workspace_size(T, 1, 16, 32, 128) > cap
    g = prefill_inputs([8], seed=3, with_state=False).to(dev)
    P, *_rest = _prefill_marshal(*g.args(), None, None, with_workspace=False)
    P.total_tokens = T  # sizes only: the check fails before any launch
    rc = lib.gdn_prefill_launch_noalloc(ctypes.byref(P), None)
    assert rc == _lib.GDN_EWORKSPACE
    assert "static scratch" in _lib.last_error()


def test_noalloc_in_graph_after_eager_call(dev):
    """After an eager call on the device, a noalloc prefill captured into a HIP graph
    replays bit-identically to the eager result (three replays, eager noalloc calls on
    other inputs between them)."""
    lib = _lib.load()
    inp, eo, en = _both(dev, [700, 64, 1], 21, True)  # eager noalloc call first
    g = inp.to(dev)
    out, ns = torch.full_like(eo, 3.0), torch.full_like(en, 3.0)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        P, _, _, copy_back, keep, stream = _prefill_marshal(*g.args(), out, ns,
                                                            with_workspace=False)
        rc = lib.gdn_prefill_launch_noalloc(ctypes.byref(P), ctypes.c_void_p(stream.cuda_stream))
    assert rc == _lib.GDN_OK, _lib.last_error()
    for r in range(3):
        out.fill_(3.0)
        ns.fill_(3.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        print(f"[noalloc graph] replay {r}: {torch.equal(out, eo)} {torch.equal(ns, en)}",
              flush=True)
        assert torch.equal(out, eo) and torch.equal(ns, en), f"replay {r} differs"
        _both(dev, [90, 200], 30 + r, False)  # other calls overwrite the scratch


def test_noalloc_fresh_process_capture_and_memory():
    """In a child process with no earlier noalloc call: a first call inside a capture
    returns GDN_EINVAL with a clear message and takes no memory; the first eager call
    takes the 96 MiB scratch (a decode and a workspace prefill before it did not); a
    capture after it replays bit-identically."""
    script = os.path.join(os.path.dirname(os.path.abspath(__file__)), "noalloc_fresh_process.py")
    print("[noalloc fresh process] starting child", flush=True)
    res = subprocess.run([sys.executable, script], capture_output=True, text=True, timeout=240)
    print(res.stdout[-2000:], res.stderr[-2000:], flush=True)
    assert res.returncode == 0
    r = json.loads(res.stdout.strip().splitlines()[-1])
    cap = 96 << 20
    assert r["first_in_capture_rc"] == _lib.GDN_EINVAL
    assert "before capturing" in r["first_in_capture_msg"]
    assert r["free_before"] - r["free_after_refused"] < cap // 2
    taken = r["free_before"] - r["free_after_first_call"]
    print(f"[noalloc fresh process] first call took {taken / 2**20:.1f} MiB", flush=True)
    assert cap <= taken < cap + (16 << 20)
    assert r["eager_rc"] == 0 and r["capture_rc"] == 0
    assert r["replays_bitwise"] == [True, True, True]

