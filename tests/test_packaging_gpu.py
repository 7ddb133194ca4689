"""The packed solution computes on the GPU: pack_solution() is written out to a fresh
directory, its kernel.py is imported the way a flashinfer-bench harness imports an
entry point (gdn_decode/scripts/pack_solution.py:34-82, README.md:227-257), and a
destination-passing call -- inputs positionally, then the preallocated outputs -- is
checked against the oracle.

Nothing built is copied in: the unpacked solution carries sources only (each packed HIP
source and header is checked byte-identical to the repository's), and importing its
kernel.py builds libgdn_hip.so and the fast path next to them, as the reference's
pipeline would (FAQ.md:138)."""
import importlib.util
import os
import sys

import numpy as np
import pytest
import torch

from gdn_hip import build as repo_build
from gdn_hip import pack
from gdn_hip.inputs import decode_inputs, prefill_inputs, varlen_lengths
from gdn_hip.parity import check_output, check_state
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu


def _unpack(name, dst):
    doc = pack.pack_solution(name)
    for src in doc["sources"]:
        path = dst / src["path"]
        path.parent.mkdir(parents=True, exist_ok=True)
        path.write_text(src["content"])
        if src["path"].startswith(("csrc/", "include/")):
            repo_file = os.path.join(repo_build.CSRC if src["path"].startswith("csrc/")
                                     else repo_build.INCLUDE, os.path.basename(src["path"]))
            with open(repo_file) as fh:
                assert fh.read() == src["content"], f"{src['path']} differs from the repository"
    assert not (dst / "gdn_hip" / "libgdn_hip.so").exists()
    return doc


def _import_entry(dst, name, entry):
    """Import dst/kernel.py with the packed gdn_hip package (not the repository's)."""
    saved = {k: v for k, v in sys.modules.items() if k == "gdn_hip" or k.startswith("gdn_hip.")}
    for k in saved:
        del sys.modules[k]
    saved_path = list(sys.path)
    try:
        spec = importlib.util.spec_from_file_location(f"packed_{name}_kernel", dst / "kernel.py")
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        fn = getattr(mod, entry)
        pkg = sys.modules["gdn_hip"]
        assert os.path.dirname(pkg.__file__) == str(dst / "gdn_hip")
        assert sys.modules["gdn_hip._lib"].LIB_PATH == str(dst / "gdn_hip" / "libgdn_hip.so")
        assert (dst / "gdn_hip" / "libgdn_hip.so").exists()  # built by the import
        return fn
    finally:
        for k in [k for k in sys.modules if k == "gdn_hip" or k.startswith("gdn_hip.")]:
            del sys.modules[k]
        sys.modules.update(saved)
        sys.path[:] = saved_path


@pytest.mark.timeout(600)
def test_packed_decode_dps(dev, tmp_path):
    doc = _unpack("gdn_decode", tmp_path)
    assert doc["definition"] == "gdn_decode_qk4_v8_d128_k_last"
    fn = _import_entry(tmp_path, "gdn_decode", doc["spec"]["entry_point"].split("::")[1])
    inp = decode_inputs(16, hqk=4, hv=8, seed=2024)
    ref_o, ref_s = O.decode(*inp.args())
    g = inp.to(dev)
    out = torch.full_like(g.v, 3.0)
    ns = torch.full_like(g.state, 3.0)
    ret = fn(*g.args(), out, ns)  # DPS: outputs appended after the inputs
    torch.cuda.synchronize()
    assert ret[0].data_ptr() == out.data_ptr() and ret[1].data_ptr() == ns.data_ptr()
    vo, vs = check_output(out, ref_o), check_state(ns, ref_s)
    print(f"[packed gdn_decode] output {vo} | state {vs}", flush=True)
    assert vo.ok and vs.ok


@pytest.mark.timeout(600)
def test_packed_prefill_dps(dev, tmp_path):
    doc = _unpack("gdn_prefill", tmp_path)
    assert doc["definition"] == "gdn_prefill_qk4_v8_d128_k_last"
    fn = _import_entry(tmp_path, "gdn_prefill", doc["spec"]["entry_point"].split("::")[1])
    lens = varlen_lengths(6, seed=11)
    inp = prefill_inputs(lens, hqk=4, hv=8, seed=11, with_state=True)
    ref_o, ref_s = O.prefill(*inp.args())
    g = inp.to(dev)
    out = torch.full((g.q.shape[0], 8, 128), 3.0, dtype=torch.bfloat16, device=dev)
    ns = torch.full_like(g.state, 3.0)
    fn(*g.args(), out, ns)
    torch.cuda.synchronize()
    vo, vs = check_output(out, ref_o), check_state(ns, ref_s)
    print(f"[packed gdn_prefill] lens={lens} output {vo} | state {vs}", flush=True)
    assert vo.ok and vs.ok
    assert np.isfinite(out.float().cpu().numpy()).all()
