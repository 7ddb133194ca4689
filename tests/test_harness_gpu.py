"""The flashinfer-bench-style harness (tests/harness.py) on a few workloads: every
record is PASSED and carries the results-file fields."""
import os
import sys

import pytest

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

pytestmark = pytest.mark.gpu


def test_harness_quick_records(dev):
    import harness

    wl = harness.workloads(quick=True)
    picked = [w for w in wl if w[1] in ("decode_b16", "prefill_varlen8")]
    assert len(picked) == 2
    results = {}
    for defn, name, kind, inp in picked:
        rec = harness.run_workload(kind, inp, dev)
        print(defn, name, rec, flush=True)
        results.setdefault(defn, {})[name] = rec
        assert rec["status"] == "PASSED"
        for f in ("latency_ms", "reference_latency_ms", "speedup_factor", "max_abs_error",
                  "max_rel_error"):
            assert f in rec
    assert all(v > 0 for v in harness.kernel_scores(results).values())


def test_harness_gate_zeroes_failed_kernel():
    import harness

    res = {"d": {"a": {"status": "PASSED", "speedup_factor": 3.0},
                 "b": {"status": "INCORRECT_NUMERICAL", "speedup_factor": 9.0}}}
    assert harness.kernel_scores(res) == {"d": 0.0}
