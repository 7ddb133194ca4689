"""CPU tests of the solution packaging (gdn_decode/scripts/pack_solution.py:34-82
contract): the packed JSON carries the reference's metadata fields and sources that
build and import on their own, outside the repository layout."""
import json
import os
import subprocess
import sys

import pytest

from gdn_hip import pack
from gdn_hip._lib import EXPORTED


@pytest.mark.parametrize("name,entry", [("gdn_decode", "kernel.py::gdn_decode"),
                                        ("gdn_prefill", "kernel.py::gdn_prefill")])
def test_pack_metadata(name, entry):
    doc = pack.pack_solution(name)
    assert doc["definition"] == f"{name}_qk4_v8_d128_k_last"
    assert doc["spec"]["entry_point"] == entry
    assert doc["spec"]["destination_passing_style"] is True
    paths = {s["path"] for s in doc["sources"]}
    assert {"kernel.py", "gdn_hip/api.py", "csrc/gdn_prefill.hip", "csrc/gdn_prefill.h",
            "csrc/gdn_prefill_plan.hip", "csrc/gdn_prefill_prep.hip", "csrc/gdn_prefill_scan.hip",
            "include/gdn_hip.h"} <= paths
    assert not any(p.startswith("oracle") for p in paths)  # the oracle never ships
    json.dumps(doc)


def test_packed_solution_builds_on_import(tmp_path):
    """The reference pipeline packs sources only and imports the entry point
    (gdn_decode/scripts/pack_solution.py:34-82, FAQ.md:138): the first import of the
    unpacked solution builds libgdn_hip.so and the fast-path extension next to the
    sources, and a second import builds nothing."""
    doc = pack.pack_solution("gdn_prefill")
    for src in doc["sources"]:
        dst = tmp_path / src["path"]
        dst.parent.mkdir(parents=True, exist_ok=True)
        dst.write_text(src["content"])
    assert not os.path.exists(tmp_path / "gdn_hip" / "libgdn_hip.so")
    code = ("import sys, ctypes; sys.path.insert(0, %r); import kernel; "
            "from gdn_hip import build; lib = ctypes.CDLL(build.LIB_PATH); "
            "print(all(hasattr(lib, s) for s in %r), kernel.gdn_prefill.__name__, "
            "build.fast_lib_path() is not None)" % (str(tmp_path), list(EXPORTED)))
    res = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                         timeout=900, cwd=str(tmp_path))
    assert res.returncode == 0, res.stderr[-2000:]
    assert res.stdout.split() == ["True", "gdn_prefill", "True"]
    assert "building" in res.stderr
    lib_path = tmp_path / "gdn_hip" / "libgdn_hip.so"
    mtime = os.path.getmtime(lib_path)
    res = subprocess.run([sys.executable, "-c", "import sys; sys.path.insert(0, %r); "
                          "import kernel" % str(tmp_path)], capture_output=True, text=True,
                         timeout=300, cwd=str(tmp_path))
    assert res.returncode == 0, res.stderr[-2000:]
    assert "building" not in res.stderr and os.path.getmtime(lib_path) == mtime


def test_solution_language_is_one_the_reference_lists():
    """FAQ.md:53-56 maps language = "python" to solution/python/ (next to triton and
    cuda), and FAQ.md:138 points kernels with their own build at a Python solution."""
    for name in ("gdn_decode", "gdn_prefill"):
        assert pack.pack_solution(name)["spec"]["language"] in ("python", "triton", "cuda")
