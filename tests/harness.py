"""Per-workload benchmark + correctness harness with flashinfer-bench's contract.

Test infrastructure (it runs the CPU oracle as the reference). It reproduces what
the reference's drivers and their external harness do for this path:

* workloads per definition, each called destination-passing style with
  preallocated ``output`` / ``new_state`` (README.md:227-257);
* correctness: an element fails only if both ``|err| > atol`` and ``|err| > rtol |ref|``,
  a workload passes at matched ratio 1.0 (FAQ.md:104-110); output at the contest's
  atol = rtol = 1e-2, new_state at the tighter bar this path is held to (elementwise
  rtol 1e-3 / atol 1e-4 and normwise 1e-3, gdn_hip.parity);
* timing: warmup / iterations / trials = 3 / 100 / 5 for decode and 1 / 10 / 3 for
  prefill (gdn_decode/scripts/run_local.py:33, gdn_prefill/scripts/run_local.py:33),
  median trial, HIP events on the launch stream;
* records {status, solution, latency_ms, reference_latency_ms, speedup_factor,
  max_abs_error, max_rel_error} (gdn_decode/scripts/run_local.py:61-74) in the
  results-file layout (gdn_decode/results/*.json:1-10); ``reference_latency_ms`` is
  the CPU oracle's time on this host;
* the scoring gate: any failing workload zeroes that kernel's score
  (computer_track_scores_local.py:157-158).

    python tests/harness.py [--out harness.json] [--quick] [--filter SUBSTR]
    python tests/harness.py --render-md harness.json
"""
from __future__ import annotations

import argparse
import datetime
import json
import os
import statistics
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
for _p in (REPO, os.path.join(REPO, "mlsys26-flashinfer-ai-kernel-generation-contest_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

from gdn_hip import gdn_decode, gdn_prefill  # noqa: E402
from gdn_hip.inputs import decode_inputs, prefill_inputs, varlen_lengths  # noqa: E402
from gdn_hip.parity import check_output, check_state  # noqa: E402
from oracle import gdn_oracle as O  # noqa: E402

SOLUTION = "mi355x-hip"
DECODE_CFG = dict(warmup_runs=3, iterations=100, num_trials=5)
PREFILL_CFG = dict(warmup_runs=1, iterations=10, num_trials=3)


def workloads(quick=False):
    """(definition, workload name, kind, inputs) tuples."""
    wl = []
    for B in ((1, 16, 64) if quick else (1, 4, 8, 16, 32, 48, 64)):
        wl.append(("gdn_decode_qk4_v8_d128_k_last", f"decode_b{B}", "decode",
                   decode_inputs(B, hqk=4, hv=8, seed=1000 + B)))
    for B in ((1, 64) if quick else (1, 64, 256)):
        wl.append(("gdn_decode_qk16_v32_d128_k_last", f"decode_b{B}", "decode",
                   decode_inputs(B, seed=B)))
    pre4 = [("prefill_varlen8", varlen_lengths(8, seed=7)), ("prefill_1x1024", [1024])]
    if not quick:
        pre4 += [("prefill_varlen16", varlen_lengths(16, seed=3)), ("prefill_1x4096", [4096]),
                 ("prefill_varlen24", varlen_lengths(24, seed=5)), ("prefill_1x256", [256])]
    for name, lens in pre4:
        wl.append(("gdn_prefill_qk4_v8_d128_k_last", name, "prefill",
                   prefill_inputs(lens, hqk=4, hv=8, seed=len(lens), with_state=True)))
    pre16 = [("prefill_4k_zero_state", [4096], False)]
    if not quick:
        pre16 += [("prefill_varlen16_8k", varlen_lengths(16, seed=0), True)]
    for name, lens, st in pre16:
        wl.append(("gdn_prefill_qk16_v32_d128_k_last", name, "prefill",
                   prefill_inputs(lens, seed=0, with_state=st)))
    return wl


def _time_gpu(fn, cfg):
    for _ in range(cfg["warmup_runs"]):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    trials = []
    for _ in range(cfg["num_trials"]):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record(stream)
        for _ in range(cfg["iterations"]):
            fn()
        e.record(stream)
        torch.cuda.synchronize()
        trials.append(s.elapsed_time(e) / cfg["iterations"])
    return statistics.median(trials)


def run_workload(kind, inp, dev):
    if kind == "decode":
        t0 = time.perf_counter()
        ref_out, ref_ns = O.decode(*inp.args())
        ref_ms = (time.perf_counter() - t0) * 1e3
        g = inp.to(dev)
        out = torch.empty_like(g.v)
        ns = torch.empty((g.q.shape[0], g.v.shape[2], 128, 128), dtype=torch.float32,
                         device=dev)
        call = lambda: gdn_decode(*g.args(), out, ns)  # noqa: E731  (DPS: outputs last)
        cfg = DECODE_CFG
    else:
        t0 = time.perf_counter()
        ref_out, ref_ns = O.prefill(*inp.args())
        ref_ms = (time.perf_counter() - t0) * 1e3
        g = inp.to(dev)
        out = torch.empty((g.q.shape[0], g.v.shape[1], 128), dtype=torch.bfloat16, device=dev)
        ns = torch.empty((len(inp.seqlens), g.v.shape[1], 128, 128), dtype=torch.float32,
                         device=dev)
        call = lambda: gdn_prefill(*g.args(), out, ns)  # noqa: E731
        cfg = PREFILL_CFG
    try:
        call()
        torch.cuda.synchronize()
    except Exception as exc:  # the harness reports, it does not raise
        return dict(status="RUNTIME_ERROR", solution=SOLUTION, error=str(exc))
    vo = check_output(out, ref_out)
    vs = check_state(ns, ref_ns)
    status = "PASSED" if (vo.ok and vs.ok) else "INCORRECT_NUMERICAL"
    lat = _time_gpu(call, cfg)
    rec = dict(status=status, solution=SOLUTION, latency_ms=lat, reference_latency_ms=ref_ms,
               speedup_factor=ref_ms / lat if lat > 0 else None,
               max_abs_error=max(vo.max_abs, vs.max_abs),
               max_rel_error=max(vo.max_rel, vs.max_rel),
               output_max_abs_error=vo.max_abs, state_norm_rel_error=vs.norm_rel)
    if kind == "decode":
        # the same launch pre-marshalled (no per-call validation): what the kernel costs
        from gdn_hip.api import DecodePlan
        plan = DecodePlan(*g.args(), out, ns)
        rec["prevalidated_latency_ms"] = _time_gpu(plan.run, cfg)
    return rec


def kernel_scores(results):
    """Mean speedup per definition, zeroed if any workload failed."""
    scores = {}
    for defn, entries in results.items():
        ok = all(e["status"] == "PASSED" for e in entries.values())
        sp = [e["speedup_factor"] for e in entries.values() if e.get("speedup_factor")]
        scores[defn] = (sum(sp) / len(sp)) if (ok and sp) else 0.0
    return scores


def render_md(doc, json_name):
    """Markdown rendering of a results document (the table of profiles/harness_workloads.md)."""
    lines = [
        "# Per-workload records of tests/harness.py (flashinfer-bench record fields)", "",
        "MI355X, one GPU. Commands (from the repository root): `python tests/harness.py --out "
        f"gpurun_out/harness.json`, then `python tests/harness.py --render-md "
        f"gpurun_out/harness.json`. The JSON document is committed beside this file as "
        f"`{json_name}`, in the reference's results-file layout "
        "(gdn_decode/results/*.json: solution_name, definition(s), timestamp, gpu, "
        "benchmark_config, results per definition and workload).", "",
        "Decode: warmup 3 / 100 iterations / 5 trials; prefill: 1 / 10 / 3 "
        "(gdn_decode/scripts/run_local.py:33, gdn_prefill/scripts/run_local.py:33), median "
        "trial, HIP events on the launch stream. `latency` is the public entry point called "
        "destination-passing style, host cost included; `prevalidated` is the same launch "
        "through a pre-marshalled `DecodePlan`. `reference` is the float64 CPU oracle on the "
        "host. Status: output within atol = rtol = 1e-2 and new_state within rtol 1e-3 / atol "
        "1e-4 elementwise and 1e-3 normwise.", "",
        "Like flashinfer-bench, every iteration of a workload reuses one set of buffers, so "
        "working sets below the 256 MB Infinity Cache (e.g. qk4_v8 decode at B=64: 64 MiB) stay "
        "resident between iterations: these latencies are not HBM figures (bench.py rotates "
        "buffer sets for that).", "",
        f"GPU: {doc['gpu']}; timestamp {doc['timestamp']}.", "",
        "| definition | workload | status | latency us | prevalidated us | reference ms | "
        "speedup | output max abs err | state norm rel err |",
        "|---|---|---|---|---|---|---|---|---|"]
    for defn, ents in doc["results"].items():
        for name, e in ents.items():
            pv = e.get("prevalidated_latency_ms")
            pvs = "" if pv is None else f"{pv * 1e3:.2f}"
            lines.append(f"| {defn} | {name} | {e['status']} | {e['latency_ms'] * 1e3:.2f} | "
                         f"{pvs} | {e['reference_latency_ms']:.2f} | {e['speedup_factor']:.0f} | "
                         f"{e['output_max_abs_error']:.1e} | {e['state_norm_rel_error']:.1e} |")
    lines += ["", "Kernel scores (mean speedup per definition, zeroed by any failed workload, "
              "computer_track_scores_local.py:157-158): "
              + ", ".join(f"{k} {v:.0f}" for k, v in doc["kernel_scores"].items())]
    return "\n".join(lines) + "\n"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", default=None)
    ap.add_argument("--render-md", metavar="RESULTS_JSON", default=None,
                    help="print the markdown table of a results document and exit")
    ap.add_argument("--quick", action="store_true")
    ap.add_argument("--filter", default="",
                    help="run only workloads whose '<definition>/<workload>' contains this")
    args = ap.parse_args()
    if args.render_md:
        with open(args.render_md) as f:
            sys.stdout.write(render_md(json.load(f), "harness_workloads.json"))
        return
    if not torch.cuda.is_available():
        print("harness: no HIP device", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda", 0)
    results = {}
    for defn, name, kind, inp in workloads(args.quick):
        if args.filter not in f"{defn}/{name}":
            continue
        print(f"[harness] {defn} {name} ...", flush=True)
        rec = run_workload(kind, inp, dev)
        results.setdefault(defn, {})[name] = rec
        print(f"[harness]   {rec['status']} latency {rec.get('latency_ms', float('nan')):.4f} ms "
              f"max_abs {rec.get('max_abs_error', float('nan')):.2e}", flush=True)
    doc = {
        "solution_name": SOLUTION,
        "timestamp": datetime.datetime.now().strftime("%Y%m%d_%H%M%S"),
        "gpu": torch.cuda.get_device_name(dev),
        "benchmark_config": {"decode": DECODE_CFG, "prefill": PREFILL_CFG},
        "results": results,
        "kernel_scores": kernel_scores(results),
    }
    text = json.dumps(doc, indent=2)
    if args.out:
        os.makedirs(os.path.dirname(os.path.abspath(args.out)), exist_ok=True)
        with open(args.out, "w") as f:
            f.write(text)
    print(json.dumps(doc["kernel_scores"]), flush=True)
    failed = [n for d in results.values() for n, e in d.items() if e["status"] != "PASSED"]
    sys.exit(1 if failed else 0)


if __name__ == "__main__":
    main()
