"""Benchmark of the GDN decode / prefill HIP path on one MI355X.

Prints ONE JSON line. Headline (``value``): decode at 64 sequences x 1 token
(16 q/k heads, 32 v heads, D = 128, fp32 k-last state) as algorithmic HBM GB/s,
timed with HIP events on the launch stream over K back-to-back steps. A step is
one decode over the whole batch; four distinct buffer sets rotate so that the
256 MiB working set of one step cannot stay resident in the 256 MB Infinity
Cache between steps. Beside it: ``decode_b1`` (1 sequence, the latency case),
``decode_b256_inplace`` (256 sequences, state updated in place), ``prefill`` (16
sequences, lengths ~ U[64, 1024] from seed 0, non-zero initial state) and
``prefill_single_4k`` (one 4096-token sequence, zero state), the prefills as Mtok/s and
algorithmic bf16 MFMA TFLOP/s. ``cpu_baseline`` times the fp32 CPU oracle on the host
cores over a bounded sample of the headline workload; ``cpu_baseline_more`` does the
same for the 1-sequence decode and the 16-sequence prefill.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
    python bench.py --trace-summary <rocprofv3 kernel_trace.csv> [--skip-first N]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.join(REPO, "mlsys26-flashinfer-ai-kernel-generation-contest_amd")
for _p in (REPO, PKG_ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = "decode us/step + HBM GB/s @B=64; prefill Mtok/s + MFMA util @8K tokens"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _traffic_from_profile(name):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE,
    scaled by the copy-kernel calibration), read from profiles/<name>; None if absent."""
    path = os.path.join(REPO, "profiles", name)
    try:
        with open(path) as f:
            for ln in f:
                if ln.startswith("traffic_bytes_per_launch:"):
                    return int(float(ln.split(":", 1)[1].strip()))
    except OSError:
        pass
    return None


def bench_decode(steps, warmup, batch=64, nsets=4, inplace=False):
    """Decode over `nsets` rotating buffer sets (pre-marshalled DecodePlans, HIP events
    on the launch stream); `inplace`: new_state is the state buffer itself."""
    import torch

    from gdn_hip.api import DecodePlan
    from gdn_hip.inputs import decode_bytes, decode_inputs

    dev = torch.device("cuda", 0)
    base = decode_inputs(batch, seed=0).to(dev)
    plans = []
    for i in range(nsets):
        st = base.state.clone()
        plans.append(DecodePlan(base.q.clone(), base.k.clone(), base.v.clone(), st,
                                base.A_log, base.a.clone(), base.dt_bias, base.b.clone(),
                                base.scale, torch.empty_like(base.v),
                                st if inplace else torch.empty_like(st)))
    del base
    stream = torch.cuda.current_stream(dev)
    for i in range(warmup):
        plans[i % nsets].run()
    torch.cuda.synchronize()
    trials = []
    for _ in range(3):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(stream)
        for i in range(steps):
            plans[i % nsets].run()
        end.record(stream)
        torch.cuda.synchronize()
        trials.append(start.elapsed_time(end) / steps)  # ms per step
    ms = statistics.median(trials)
    nbytes = decode_bytes(batch)
    gbs = nbytes / (ms * 1e-3) / 1e9
    del plans
    torch.cuda.empty_cache()
    return dict(ms=ms, gbs=gbs, bytes=nbytes, trials=trials)


def bench_prefill(steps, warmup, lens=None, with_state=True, settle_ms=0.0):
    """Prefill over `lens` (default: 16 sequences, lengths ~U[64,1024] from seed 0).

    `warmup` calls, then back-to-back calls for at least `settle_ms` of GPU time before the
    timed trials: under this sustained MFMA and HBM load the clock management runs the first
    ~100-200 calls slower (up to ~25 % at 8172 tokens) before it settles
    (profiles/prefill_clock_curve.md), and a serving loop runs in the settled state."""
    import torch

    from gdn_hip import gdn_prefill
    from gdn_hip.inputs import prefill_flops, prefill_inputs, varlen_lengths

    dev = torch.device("cuda", 0)
    lens = lens or varlen_lengths(16, seed=0)
    inp = prefill_inputs(lens, seed=0, with_state=with_state).to(dev)
    T = sum(lens)
    out = torch.empty((T, 32, 128), dtype=torch.bfloat16, device=dev)
    ns = torch.empty((len(lens), 32, 128, 128), dtype=torch.float32, device=dev)
    for _ in range(warmup):
        gdn_prefill(*inp.args(), output=out, new_state=ns)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    settled = 0.0
    while settled < settle_ms:
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record(stream)
        for _ in range(20):
            gdn_prefill(*inp.args(), output=out, new_state=ns)
        s1.record(stream)
        torch.cuda.synchronize()
        settled += s0.elapsed_time(s1)
    trials = []
    for _ in range(3):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(steps):
            gdn_prefill(*inp.args(), output=out, new_state=ns)
        end.record(stream)
        torch.cuda.synchronize()
        trials.append(start.elapsed_time(end) / steps)
    ms = statistics.median(trials)
    flops = prefill_flops(T)
    tflops = flops / (ms * 1e-3) / 1e12
    return dict(tokens=T, nseqs=len(lens), ms=ms, mtok_s=T / (ms * 1e-3) / 1e6, tflops=tflops,
                mfma_frac=tflops / BF16_PEAK_TFLOPS, settle_ms=round(settled, 1), trials=trials)


def prefill_curve(batches, lens=None, with_state=True):
    """us/call of back-to-back prefills, per batch of 20 calls, from the process's first
    call on: how the clock management settles under this load."""
    import torch

    from gdn_hip import gdn_prefill
    from gdn_hip.inputs import prefill_inputs, varlen_lengths

    dev = torch.device("cuda", 0)
    lens = lens or varlen_lengths(16, seed=0)
    inp = prefill_inputs(lens, seed=0, with_state=with_state).to(dev)
    T = sum(lens)
    out = torch.empty((T, 32, 128), dtype=torch.bfloat16, device=dev)
    ns = torch.empty((len(lens), 32, 128, 128), dtype=torch.float32, device=dev)
    gdn_prefill(*inp.args(), output=out, new_state=ns)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(batches + 1)]
    ev[0].record(stream)
    for b in range(batches):
        for _ in range(20):
            gdn_prefill(*inp.args(), output=out, new_state=ns)
        ev[b + 1].record(stream)
    torch.cuda.synchronize()
    us = [ev[i].elapsed_time(ev[i + 1]) / 20 * 1e3 for i in range(batches)]
    print(json.dumps({"workload": f"prefill T={T} ({len(lens)} sequences)",
                      "us_per_call_per_batch_of_20": [round(x, 1) for x in us]}), flush=True)


def _host_cores():
    """(threads used, cores this process may run on, cores of the host)."""
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return max(1, min(avail, 16)), avail, os.cpu_count() or avail


def _time_cpu(fn, budget_s, max_n=200):
    fn()  # warm
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= max_n:
            return el / n, n


def cpu_baseline_decode(batch=64, budget_s=10.0, max_n=1000):
    """Time the float32 C oracle (a port of the reference arithmetic) on the host cores
    over repeated full decode steps, up to ~budget_s seconds or max_n steps."""
    from gdn_hip.inputs import decode_bytes, decode_inputs
    from oracle import gdn_oracle as O

    cores, avail, total = _host_cores()
    inp = decode_inputs(batch, seed=0)
    args = (inp.q, inp.k, inp.v, inp.state, inp.A_log, inp.a, inp.dt_bias, inp.b, inp.scale)
    sec, n = _time_cpu(lambda: O.decode(*args, precision="f32", threads=cores), budget_s,
                       max_n=max_n)
    return dict(value=decode_bytes(batch) / sec / 1e9, unit="GB/s", cores=cores,
                cores_available=avail, cores_host=total, kind="port",
                us_per_step=sec * 1e6,
                sample=f"{n} full decode steps (B={batch}, fp32 C oracle, OpenMP over "
                       f"(sequence, v-head)); {sec * 1e3:.2f} ms/step")


def cpu_baseline_prefill(budget_s=5.0):
    """The fp32 C oracle on the whole 16-sequence prefill (token recurrence, OpenMP over
    (sequence, v-head)), repeated up to ~budget_s seconds."""
    from gdn_hip.inputs import prefill_inputs, varlen_lengths
    from oracle import gdn_oracle as O

    cores, avail, total = _host_cores()
    lens = varlen_lengths(16, seed=0)
    inp = prefill_inputs(lens, seed=0, with_state=True)
    sec, n = _time_cpu(lambda: O.prefill(*inp.args(), precision="f32", threads=cores),
                       budget_s, max_n=50)
    T = sum(lens)
    return dict(value=T / sec / 1e6, unit="Mtok/s", cores=cores, cores_available=avail,
                cores_host=total, kind="port", us_per_step=sec * 1e6,
                sample=f"{n} full prefills (16 sequences, T={T}, fp32 C oracle); "
                       f"{sec * 1e3:.1f} ms/step")


def summarize_trace(path, skip_first=0, last=0):
    """Per-kernel dispatch durations from a rocprofv3 kernel_trace.csv, dropping each
    kernel's first `skip_first` dispatches (the warmup calls), or keeping only its `last`
    ones (the timed calls after the prefill's settling phase); prints a markdown table."""
    import csv
    from collections import defaultdict

    per = defaultdict(list)
    with open(path) as f:
        for row in csv.DictReader(f):
            per[row["Kernel_Name"]].append((int(row["Start_Timestamp"]),
                                            int(row["End_Timestamp"]) - int(row["Start_Timestamp"])))
    per = {k: [d for _, d in sorted(v)] for k, v in per.items()}
    sel = (lambda d: d[-last:]) if last > 0 else (lambda d: d[skip_first:])
    what = f"the last {last}" if last > 0 else f"after skipping {skip_first}"
    print(f"| kernel | dispatches ({what}) | avg us | min us | max us |")
    print("|---|---|---|---|---|")
    for name, d in sorted(per.items(), key=lambda kv: -sum(sel(kv[1]))):
        d = sel(d)
        if not d:
            continue
        short = name.split("(")[0][:90]
        print(f"| `{short}` | {len(d)} | {sum(d) / len(d) / 1e3:.2f} | {min(d) / 1e3:.2f} | "
              f"{max(d) / 1e3:.2f} |")


def summarize_pmc(fetch_csv, write_csv, skip_first=0, algo_bytes=None, title=""):
    """HBM traffic per kernel from two rocprofv3 --pmc runs (FETCH_SIZE, then WRITE_SIZE;
    counter_collection.csv of each), scaled by what the same counters read for the
    268,435,456-byte device copy of --calibrate-copy in those runs; prints the summary
    that profiles/*_traffic.txt hold, ending in a traffic_bytes_per_launch line."""
    import csv
    from collections import defaultdict

    vals = defaultdict(lambda: defaultdict(list))
    for path in (fetch_csv, write_csv):
        with open(path) as f:
            for row in csv.DictReader(f):
                vals[row["Kernel_Name"]][row["Counter_Name"]].append(float(row["Counter_Value"]))
    # calibration kernel: torch's elementwise multiply of --calibrate-copy (its own kernel:
    # reads 256 MiB, writes 256 MiB); the runtime's copy kernel is listed beside it
    ref = next((k for k in vals if "elementwise" in k and "MulFunctor" in k), None)
    if ref is None:
        ref = next((k for k in vals if "elementwise" in k), None)
    if ref is None:
        raise SystemExit("no calibration kernel in the counter files: run with --calibrate-copy")
    copy_bytes = 268435456
    avg = lambda k, c: sum(vals[k][c]) / len(vals[k][c])  # noqa: E731
    fk, wk = avg(ref, "FETCH_SIZE"), avg(ref, "WRITE_SIZE")
    rf, wf = copy_bytes / (fk * 1024), copy_bytes / (wk * 1024)
    print(f"# {title}".rstrip())
    print(f"# Calibration: an elementwise multiply over {copy_bytes:,} bytes reads FETCH_SIZE = "
          f"{fk:,.1f} KiB and writes WRITE_SIZE = {wk:,.1f} KiB")
    print(f"#   => read factor {rf:.3f}, write factor {wf:.3f} (bytes per counted KiB / 1024)")
    for k in vals:
        if "copyBuffer" in k:
            print(f"#   (the runtime's copy kernel of the same size reads FETCH_SIZE = "
                  f"{avg(k, 'FETCH_SIZE'):,.1f} KiB, writes WRITE_SIZE = {avg(k, 'WRITE_SIZE'):,.1f} KiB)")
    print(f"# averages per dispatch over the timed calls (first {skip_first} dispatches of each "
          "kernel dropped)")
    print("#")
    print(f"# {'kernel':40s} {'dispatches':>10s} {'FETCH KiB':>12s} {'bytes read':>14s} "
          f"{'WRITE KiB':>12s} {'bytes written':>14s}")
    total = 0.0
    for name, c in sorted(vals.items()):
        if name == ref or "fillBuffer" in name or "copyBuffer" in name or "elementwise" in name:
            continue
        fv, wv = c.get("FETCH_SIZE", [])[skip_first:], c.get("WRITE_SIZE", [])[skip_first:]
        if not fv or not wv:
            continue
        f_avg, w_avg = sum(fv) / len(fv), sum(wv) / len(wv)
        rb, wb = f_avg * 1024 * rf, w_avg * 1024 * wf
        total += rb + wb
        short = name.split("(")[0].replace("void ", "")[:40]
        print(f"# {short:40s} {len(fv):10d} {f_avg:12,.1f} {rb:14,.0f} {w_avg:12,.1f} {wb:14,.0f}")
    print("#")
    print(f"# measured total per launch (all kernels above) = {total:,.0f} B")
    if algo_bytes:
        print(f"# algorithmic bytes = {algo_bytes:,} -> measured / algorithmic = "
              f"{total / algo_bytes:.2f}")
    print(f"traffic_bytes_per_launch: {int(total)}")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=10.0,
                    help="seconds of CPU work for the decode B=64 baseline (B=1 takes "
                         "0.15 of it, the prefill 0.6)")
    ap.add_argument("--prefill-settle-ms", type=float, default=40.0,
                    help="prefill lines: back-to-back calls for this much GPU time after the "
                         "warmup calls, before timing (clock settling under sustained load)")
    ap.add_argument("--only", choices=["all", "decode", "prefill", "prefill4k"], default="all",
                    help="run one path only (profiling runs)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also launch a plain 256 MiB device copy (rocprof counter calibration)")
    ap.add_argument("--trace-summary", metavar="CSV",
                    help="summarise a rocprofv3 kernel_trace.csv per kernel and exit")
    ap.add_argument("--skip-first", type=int, default=0,
                    help="with --trace-summary / --pmc-summary: dispatches to drop per kernel")
    ap.add_argument("--curve", type=int, default=0, metavar="BATCHES",
                    help="print the prefill's us/call over BATCHES back-to-back batches of 20 "
                         "calls from a cold start (--only prefill or prefill4k), and exit")
    ap.add_argument("--last", type=int, default=0,
                    help="with --trace-summary: keep only each kernel's last N dispatches")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="summarise two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) per "
                         "kernel with the copy calibration, and exit")
    ap.add_argument("--algo-bytes", type=int, default=None,
                    help="with --pmc-summary: algorithmic bytes per launch to compare against")
    ap.add_argument("--title", default="", help="with --pmc-summary: heading line")
    args = ap.parse_args()
    if args.trace_summary:
        summarize_trace(args.trace_summary, args.skip_first, args.last)
        return
    if args.pmc_summary:
        summarize_pmc(*args.pmc_summary, skip_first=args.skip_first,
                      algo_bytes=args.algo_bytes, title=args.title)
        return
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this path runs on one GPU "
              "(every (sequence, head) state is independent; see the sharding notes).",
              file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        sys.exit(1)
    from gdn_hip import _lib
    from gdn_hip.inputs import prefill_bytes

    _lib.load()
    if args.calibrate_copy:
        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
            torch.mul(src, 2.0, out=dst)  # an elementwise kernel: reads and writes 256 MiB
        torch.cuda.synchronize()
        log("copy calibration: 3 x 268435456-byte device copies and elementwise multiplies")
        del src, dst
    psteps = max(3, min(args.steps, 50))
    pwarm = 5
    if args.curve:
        lens, st = (None, True) if args.only != "prefill4k" else ([4096], False)
        prefill_curve(args.curve, lens=lens, with_state=st)
        return
    if args.only in ("prefill", "prefill4k"):
        lens, st = (None, True) if args.only == "prefill" else ([4096], False)
        pre = bench_prefill(psteps, pwarm, lens=lens, with_state=st,
                            settle_ms=args.prefill_settle_ms)
        log(f"prefill: T={pre['tokens']} {pre['ms'] * 1e3:.1f} us/step "
            f"{pre['mtok_s']:.1f} Mtok/s {pre['tflops']:.1f} TFLOP/s")
        return
    log(f"decode B=64: warmup {args.warmup}, steps {args.steps}")
    dec = bench_decode(args.steps, args.warmup)
    log(f"decode: {dec['ms'] * 1e3:.2f} us/step, {dec['gbs']:.0f} GB/s (trials {dec['trials']})")
    if args.only == "decode":
        return
    dec1 = bench_decode(args.steps, args.warmup, batch=1, nsets=16)
    log(f"decode B=1: {dec1['ms'] * 1e3:.2f} us/step")
    dec256 = bench_decode(max(10, args.steps // 4), max(2, args.warmup // 4), batch=256, nsets=2,
                          inplace=True)
    log(f"decode B=256 in place: {dec256['ms'] * 1e3:.2f} us/step, {dec256['gbs']:.0f} GB/s")
    pre = pre4k = None
    if not args.no_prefill:
        log(f"prefill 16x varlen: warmup {pwarm}, steps {psteps}")
        pre = bench_prefill(psteps, pwarm, settle_ms=args.prefill_settle_ms)
        log(f"prefill: T={pre['tokens']} {pre['ms'] * 1e3:.1f} us/step "
            f"{pre['mtok_s']:.1f} Mtok/s {pre['tflops']:.1f} TFLOP/s")
        pre4k = bench_prefill(psteps, pwarm, lens=[4096], with_state=False,
                              settle_ms=args.prefill_settle_ms)
        log(f"prefill 1x4096: {pre4k['ms'] * 1e3:.1f} us/step {pre4k['tflops']:.1f} TFLOP/s")
    cpu = cpu_more = None
    if not args.no_cpu:
        log("cpu baselines (fp32 C oracle): decode B=64, decode B=1, prefill 16x varlen")
        cpu = cpu_baseline_decode(budget_s=args.cpu_budget)
        cpu1 = cpu_baseline_decode(batch=1, budget_s=0.15 * args.cpu_budget, max_n=20000)
        cpu1.update(value=cpu1["us_per_step"], unit="us/step (lower is better)")
        cpu_more = {"decode_b1": cpu1}
        if not args.no_prefill:
            cpu_more["prefill"] = cpu_baseline_prefill(budget_s=0.6 * args.cpu_budget)
        log(f"cpu: {cpu['value']:.2f} GB/s on {cpu['cores']} of {cpu['cores_host']} cores")
    traffic = _traffic_from_profile("decode_b64_traffic.txt")
    rec = {
        "metric": METRIC,
        "value": round(dec["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded; q,k L2-normalised bf16, v/a/b N(0,1) bf16, state N(0,0.02) fp32)",
        "config": {
            "workload": "GDN decode, 64 sequences x 1 token, 16 q/k heads, 32 v heads, "
                        "D=128, fp32 k-last state (4 rotating buffer sets)",
            "batch": 64, "num_qk_heads": 16, "num_v_heads": 32, "head_size": 128,
            "parallelism": "single GPU",
        },
        "decode_us_per_step": round(dec["ms"] * 1e3, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(dec["gbs"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dec["gbs"] / HBM_PEAK_GBS, 4),
            "traffic": traffic,
        },
        "cpu_baseline": cpu,
        "cpu_baseline_more": cpu_more,
        "decode_b1": {
            "workload": "GDN decode, 1 sequence x 1 token (16 rotating buffer sets)",
            "us_per_step": round(dec1["ms"] * 1e3, 2),
            "gb_per_s": round(dec1["gbs"], 1),
        },
        "decode_b256_inplace": {
            "workload": "GDN decode, 256 sequences x 1 token, new_state is state (2 sets)",
            "us_per_step": round(dec256["ms"] * 1e3, 2),
            "gb_per_s": round(dec256["gbs"], 1),
            "hbm_frac": round(dec256["gbs"] / HBM_PEAK_GBS, 4),
        },
    }
    if pre is not None:
        for key, r, wl, st, tfile in (
                ("prefill_single_4k", pre4k, "GDN prefill, 1 sequence x 4096 tokens, zero "
                 "initial state", False, "prefill_4k_traffic.txt"),
                ("prefill", pre, f"GDN prefill, {pre['nseqs']} sequences, lengths ~U[64,1024] "
                 f"(seed 0), T={pre['tokens']} tokens, non-zero fp32 initial state", True,
                 "prefill_varlen16_traffic.txt")):
            algo = prefill_bytes(r["tokens"], r["nseqs"], with_state=st)
            hbm = algo / (r["ms"] * 1e-3) / 1e9
            rec[key] = {
                "workload": wl,
                "us_per_step": round(r["ms"] * 1e3, 2),
                "mtok_per_s": round(r["mtok_s"], 2),
                "tflops": round(r["tflops"], 2),
                # traffic: measured HBM bytes of all kernels of one prefill (FETCH_SIZE +
                # WRITE_SIZE, copy-calibrated) against `algo_bytes`
                "roofline": {"bound": "mfma", "achieved": round(r["tflops"], 2),
                             "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(r["mfma_frac"], 4),
                             "traffic": _traffic_from_profile(tfile), "algo_bytes": algo},
                "hbm_gb_per_s": round(hbm, 1),
                "hbm_frac": round(hbm / HBM_PEAK_GBS, 4),
                "warmup_calls": pwarm,
                "settle_ms": r["settle_ms"],
            }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
