"""The C ABI called from a native C++ program (tests/native/gdn_native_caller.cpp): no
Python or torch in that process. It fills gdn_decode_params / gdn_prefill_params on
hipMalloc'd buffers and its own stream, as a C or C++ host would, and checks decode (also
in place), prefill (an empty sequence, uncovered trailing tokens, int64 cu_seqlens) and
three error codes against the float64 CPU oracle. build() compiles it."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native", "gdn_native_caller")


def test_native_cpp_caller():
    assert os.path.exists(BIN), f"{BIN} is missing: run __graft_entry__.build()"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all cases PASSED" in r.stdout
