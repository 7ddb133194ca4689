"""GPU parity of gdn_prefill (HIP, chunked WY form) against the float64 CPU oracle.

Bars (gdn_hip.parity): output bf16 atol = rtol = 1e-2 (both-condition rule of
FAQ.md:104-110); new_state fp32 elementwise rtol = 1e-3 / atol = 1e-4 and normwise
relative error <= 1e-3.
"""
import ctypes

import numpy as np
import pytest
import torch

from gdn_hip import _lib, gdn_decode, gdn_prefill, release_workspace
from gdn_hip.inputs import prefill_inputs, varlen_lengths, with_extreme_gates
from gdn_hip.parity import check_output, check_state
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu


def _oracle(inp):
    return O.prefill(inp.q, inp.k, inp.v, inp.state, inp.A_log, inp.a, inp.dt_bias, inp.b,
                     inp.cu_seqlens, inp.scale)


def _check(out, ns, ref_out, ref_ns, label):
    vo = check_output(out, ref_out)
    vs = check_state(ns, ref_ns)
    print(f"[{label}] output {vo} | state {vs}", flush=True)
    assert vo.ok, f"{label}: output {vo}"
    assert vs.ok, f"{label}: new_state {vs}"


def _run(dev, inp, label, **kw):
    print(f"[{label}] launching T={inp.q.shape[0]} lens={inp.seqlens[:8]}...", flush=True)
    ref_out, ref_ns = _oracle(inp)
    g = inp.to(dev)
    out, ns = gdn_prefill(*g.args(), **kw)
    torch.cuda.synchronize()
    _check(out, ns, ref_out, ref_ns, label)
    return g, out, ns


@pytest.mark.parametrize("lens", [[1], [5], [63], [64], [65], [128], [129], [200, 37]])
def test_prefill_small(dev, lens):
    _run(dev, prefill_inputs(lens, seed=len(lens) * 100 + lens[0], with_state=True),
         f"lens={lens}")


def test_prefill_single_4k_zero_state(dev):
    """One 4096-token sequence, zero initial state (state=None)."""
    _run(dev, prefill_inputs([4096], seed=3, with_state=False), "4k state=None")


def test_prefill_varlen_16(dev):
    """16 sequences, lengths ~U[64,1024] from the seed, non-zero fp32 initial state."""
    lens = varlen_lengths(16, seed=0)
    _run(dev, prefill_inputs(lens, seed=0, with_state=True), "varlen16")


@pytest.mark.parametrize("gates", ["mild", "none"])
def test_prefill_long_memory_gates(dev, gates):
    """alpha ~ 0.99 or exactly 1: the state carries across many chunks."""
    _run(dev, prefill_inputs([300, 700, 64], seed=5, with_state=True, gates=gates,
                             state_std=0.1), f"gates={gates}")


@pytest.mark.parametrize("hqk,hv", [(4, 8), (8, 8), (2, 8), (1, 4), (2, 6), (1, 3)])
def test_prefill_head_layouts(dev, hqk, hv):
    _run(dev, prefill_inputs([150, 90, 257], hqk=hqk, hv=hv, seed=9, with_state=True),
         f"hqk={hqk} hv={hv}")


def test_prefill_empty_sequences_and_gaps(dev):
    """Zero-length sequences keep their state; tokens outside every sequence read as
    zero output (gdn_prefill/solution/triton/kernel.py:286)."""
    _run(dev, prefill_inputs([0, 70, 0, 0, 130, 0], seed=17, with_state=True, pad_tokens=45),
         "empty+gaps")


@pytest.mark.parametrize("scale", [None, 0.0, 0.25, "host tensor", "device tensor"])
def test_prefill_scale_defaults(dev, scale):
    """scale None / 0 -> 1/sqrt(D) (gdn_prefill/solution/triton/kernel.py:276-277); a
    one-element tensor is read as its value (0.25 here). Through the Python path (no
    destination buffers), destination-passing calls (the C++ fast path for a float or None
    scale, the Python path for a tensor) and the fast path called directly, each against
    the oracle."""
    inp = prefill_inputs([150, 64, 1], hqk=4, hv=8, seed=31, with_state=True)
    inp.scale = 0.25 if isinstance(scale, str) else scale
    ref_o, ref_s = _oracle(inp)
    g = inp.to(dev)
    args = list(g.args())
    if isinstance(scale, str):
        args[-1] = torch.tensor([0.25], device=dev if scale == "device tensor" else "cpu")
    T, N = g.q.shape[0], len(inp.seqlens)
    out, ns = gdn_prefill(*args)
    o2 = torch.empty((T, 8, 128), dtype=torch.bfloat16, device=dev)
    n2 = torch.empty((N, 8, 128, 128), dtype=torch.float32, device=dev)
    gdn_prefill(*args, output=o2, new_state=n2)
    torch.cuda.synchronize()
    _check(out, ns, ref_o, ref_s, f"scale={scale}")
    _check(o2, n2, ref_o, ref_s, f"scale={scale} destination-passing")
    if not isinstance(scale, str):
        o3, n3 = torch.empty_like(o2), torch.empty_like(n2)
        assert _lib.fast().prefill(*args[:-1], 0.0 if scale is None else scale, o3, n3, 0) == 0
        torch.cuda.synchronize()
        assert torch.equal(o3, out) and torch.equal(n3, ns)


def test_prefill_int64_cu_seqlens(dev):
    _run(dev, prefill_inputs([99, 1, 250], seed=19, with_state=True, cu_dtype=torch.int64),
         "cu int64")


def test_prefill_inplace_state(dev):
    inp = prefill_inputs([180, 75], seed=23, with_state=True)
    ref_out, ref_ns = _oracle(inp)
    g = inp.to(dev)
    out, ns = gdn_prefill(*g.args(), new_state=g.state)
    torch.cuda.synchronize()
    assert ns.data_ptr() == g.state.data_ptr()
    _check(out, ns, ref_out, ref_ns, "in-place")


def test_prefill_explicit_zero_state_equals_none(dev):
    inp = prefill_inputs([333], seed=29, with_state=False).to(dev)
    o1, s1 = gdn_prefill(*inp.args())
    z = torch.zeros((1, 32, 128, 128), dtype=torch.float32, device=dev)
    args = list(inp.args())
    args[3] = z
    o2, s2 = gdn_prefill(*args)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)


def test_prefill_strided_and_preallocated(dev):
    """q/k/v as views of a fused projection; preallocated (poisoned) outputs."""
    inp = prefill_inputs([77, 160], seed=31, with_state=True)
    ref_out, ref_ns = _oracle(inp)
    g = inp.to(dev)
    T = g.q.shape[0]
    qkv = torch.empty((T, 16 + 16 + 32, 128), dtype=torch.bfloat16, device=dev)
    qkv[:, :16], qkv[:, 16:32], qkv[:, 32:] = g.q, g.k, g.v
    out = torch.full((T, 32, 128), 7.0, dtype=torch.bfloat16, device=dev)
    ns = torch.full_like(g.state, 7.0)
    o, s = gdn_prefill(qkv[:, :16], qkv[:, 16:32], qkv[:, 32:], g.state, g.A_log, g.a,
                       g.dt_bias, g.b, g.cu_seqlens, g.scale, output=out, new_state=ns)
    torch.cuda.synchronize()
    assert o.data_ptr() == out.data_ptr() and s.data_ptr() == ns.data_ptr()
    _check(o, s, ref_out, ref_ns, "strided")


def test_prefill_deterministic(dev):
    inp = prefill_inputs(varlen_lengths(8, seed=4), seed=4, with_state=True).to(dev)
    o1, s1 = gdn_prefill(*inp.args())
    o2, s2 = gdn_prefill(*inp.args())
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)


def test_prefill_no_sequences_and_no_tokens(dev):
    inp = prefill_inputs([], seed=1, with_state=True, pad_tokens=10).to(dev)
    out, ns = gdn_prefill(*inp.args())
    torch.cuda.synchronize()
    assert out.shape == (10, 32, 128) and torch.all(out == 0)
    assert ns.shape == (0, 32, 128, 128)
    inp = prefill_inputs([0, 0], seed=2, with_state=True).to(dev)
    out, ns = gdn_prefill(*inp.args())
    torch.cuda.synchronize()
    assert out.shape == (0, 32, 128) and torch.equal(ns, inp.state)


def test_prefill_resume_split(dev):
    """prefill(x[:m]) then prefill(x[m:], state) against the oracle's prefill(x): the
    state handoff between calls (k-last new_state fed back as state,
    gdn_prefill/solution/triton/kernel.py:32,288-299)."""
    inp = prefill_inputs([500], seed=37, with_state=True, gates="mild")
    ref_o, ref_s = _oracle(inp)
    g = inp.to(dev)
    m = 203
    cu1 = torch.tensor([0, m], dtype=torch.int32, device=dev)
    cu2 = torch.tensor([0, 500 - m], dtype=torch.int32, device=dev)
    o1, s1 = gdn_prefill(g.q[:m], g.k[:m], g.v[:m], g.state, g.A_log, g.a[:m],
                         g.dt_bias, g.b[:m], cu1, g.scale)
    o2, s2 = gdn_prefill(g.q[m:], g.k[m:], g.v[m:], s1, g.A_log, g.a[m:],
                         g.dt_bias, g.b[m:], cu2, g.scale)
    torch.cuda.synchronize()
    _check(torch.cat([o1, o2]), s2, ref_o, ref_s, "resume vs oracle")


def test_prefill_records_past_2gib(dev):
    """Maximum sizes: one 327,680-token sequence at 32 v-heads, whose workspace records
    (5,121 chunks x 32 v-heads x 16 KB = 2.7 GB) reach past 2^31 bytes, against the same
    sequence prefilled as five chained 65,536-token calls (0.5 GB of records each, the
    state handed from call to call). The two runs plan and cut the sequence differently,
    so they agree to rounding; an offset truncated to 32 bits in the large run would read
    or write the wrong records. Inputs are drawn on the GPU and compared there (the oracle
    would need ~0.7 TFLOP in fp64); mild decay keeps earlier chunks' states significant."""
    T, piece, hqk, hv = 5 << 16, 1 << 16, 2, 32
    g = torch.Generator(device=dev)
    g.manual_seed(61)
    unit = lambda *s: torch.nn.functional.normalize(  # noqa: E731
        torch.randn(*s, generator=g, device=dev), dim=-1).to(torch.bfloat16)
    q, k = unit(T, hqk, 128), unit(T, hqk, 128)
    v = torch.randn(T, hv, 128, generator=g, device=dev).to(torch.bfloat16)
    a = torch.randn(T, hv, generator=g, device=dev).to(torch.bfloat16)
    b = torch.randn(T, hv, generator=g, device=dev).to(torch.bfloat16)
    A_log = -6.0 + 3.0 * torch.rand(hv, generator=g, device=dev)
    dt_bias = torch.rand(hv, generator=g, device=dev) * 2.0 - 1.0
    state = torch.randn(1, hv, 128, 128, generator=g, device=dev) * 0.05
    scale = 128 ** -0.5
    ws = _lib.load().gdn_prefill_workspace_size(T, 1, hqk, hv, 128)
    print(f"[{T} tokens] whole-sequence run, workspace {ws / 2**30:.2f} GiB", flush=True)
    assert ws > (1 << 31)
    cu = torch.tensor([0, T], dtype=torch.int32, device=dev)
    o_full, s_full = gdn_prefill(q, k, v, state, A_log, a, dt_bias, b, cu, scale)
    torch.cuda.synchronize()
    cu_p = torch.tensor([0, piece], dtype=torch.int32, device=dev)
    s = state
    outs = []
    for i in range(T // piece):
        sl = slice(i * piece, (i + 1) * piece)
        o, s = gdn_prefill(q[sl], k[sl], v[sl], s, A_log, a[sl], dt_bias, b[sl], cu_p, scale)
        outs.append(o)
    torch.cuda.synchronize()
    # the output bar of gdn_hip.parity (both-condition rule), evaluated on the device
    x, y = o_full.float(), torch.cat(outs).float()
    d = (x - y).abs()
    nfail = int(((d > 1e-2) & (d > 1e-2 * y.abs())).sum())
    vs = check_state(s_full, s)
    print(f"[{T} tokens] whole vs chained: output max_abs={float(d.max()):.3e} fail={nfail} | "
          f"state {vs}", flush=True)
    assert nfail == 0 and torch.isfinite(x).all()
    assert vs.ok
    del x, y, d, o_full, outs, q, k, v
    release_workspace()


@pytest.mark.parametrize("gates", ["strong", "mild"])
def test_prefill_then_decode_matches_oracle(dev, gates):
    """Prefill's new_state feeds decode in the same k-last layout
    (gdn_prefill/solution/triton/kernel.py:32, gdn_decode/solution/triton/kernel.py:8,17):
    prefill(x) followed by four decode steps t1..t4 must equal the oracle's prefill of
    x || t1..t4, token by token and in the final state, for two sequences at once."""
    L, n_dec = [257, 64], 4
    inp = prefill_inputs([x + n_dec for x in L], seed=41, with_state=True, gates=gates)
    ref_o, ref_s = _oracle(inp)
    g = inp.to(dev)
    cu = inp.cu_seqlens.tolist()
    # prefill of the first L[i] tokens of each sequence, packed
    idx = torch.cat([torch.arange(cu[i], cu[i] + L[i]) for i in range(2)]).to(dev)
    cu_p = torch.tensor([0, L[0], L[0] + L[1]], dtype=torch.int32, device=dev)
    o_p, s = gdn_prefill(g.q[idx], g.k[idx], g.v[idx], g.state, g.A_log, g.a[idx],
                         g.dt_bias, g.b[idx], cu_p, g.scale)
    outs = []
    for j in range(n_dec):
        t = torch.tensor([cu[i] + L[i] + j for i in range(2)], device=dev)
        od, s = gdn_decode(g.q[t].unsqueeze(1), g.k[t].unsqueeze(1), g.v[t].unsqueeze(1), s,
                           g.A_log, g.a[t].unsqueeze(1), g.dt_bias, g.b[t].unsqueeze(1),
                           g.scale)
        outs.append(od[:, 0])
    torch.cuda.synchronize()
    vo = check_output(o_p, ref_o[idx.cpu().numpy()])
    print(f"[prefill part {gates}] output {vo}", flush=True)
    assert vo.ok
    dec_ref = np.stack([ref_o[[cu[i] + L[i] + j for i in range(2)]] for j in range(n_dec)],
                       axis=1)
    _check(torch.stack(outs, dim=1), s, dec_ref, ref_s, f"prefill->decode x{n_dec} {gates}")


def test_prefill_matches_exact_fixture(dev):
    """HIP prefill vs the rational-arithmetic known answers (tests/golden/make_golden.py)."""
    import os

    import numpy as np

    f = np.load(os.path.join(os.path.dirname(__file__), "golden", "gdn_kat_d128.npz"))

    def bf(x):
        return torch.from_numpy(x.view(np.int16).copy()).view(torch.bfloat16).to(dev)

    out, ns = gdn_prefill(bf(f["q"]), bf(f["k"]), bf(f["v"]), torch.from_numpy(f["state"]).to(dev),
                          torch.from_numpy(f["A_log"]).to(dev), bf(f["a"]),
                          torch.from_numpy(f["dt_bias"]).to(dev), bf(f["b"]),
                          torch.from_numpy(f["cu_seqlens"]).to(dev), float(f["scale"]))
    torch.cuda.synchronize()
    _check(out, ns, f["out"], f["new_state"], "exact fixture")


@pytest.mark.parametrize("nseq", [64, 65, 255, 300, 600])
def test_prefill_many_sequences(dev, nseq):
    """Many short and empty sequences. Up to 64 the prep kernel plans for itself (one
    sequence per lane); from 65 the planning kernel's chunk table and longest-first order
    (its sort covers up to 512 sequences) drive prep and scan."""
    g = torch.Generator().manual_seed(nseq)
    lens = [int(x) for x in torch.randint(0, 90, (nseq,), generator=g)]
    _run(dev, prefill_inputs(lens, hqk=4, hv=8, seed=nseq, with_state=True), f"N={nseq}")


@pytest.mark.parametrize("nseq", [3, 64, 300])
def test_prefill_gap_before_first_sequence(dev, nseq):
    """cu_seqlens[0] > 0: the leading tokens belong to no sequence and read as zero."""
    g = torch.Generator().manual_seed(7 + nseq)
    lens = [int(x) for x in torch.randint(1, 70, (nseq,), generator=g)]
    inp = prefill_inputs(lens, hqk=4, hv=8, seed=31, with_state=True, pad_tokens=53)
    inp.cu_seqlens = inp.cu_seqlens + 37  # 37 leading and 16 trailing gap tokens
    _run(dev, inp, f"lead gap N={nseq}")


@pytest.mark.parametrize("gates", ["strong", "mild", "none"])
def test_prefill_segments_long_memory(dev, gates):
    """Few (sequence, v-head) pairs: each long sequence is scanned as parallel segments
    whose states are chained (S_in M + R). Mild or no decay makes every segment's state
    carry into the next one."""
    _run(dev, prefill_inputs([2048], seed=41, with_state=True, gates=gates, state_std=0.1),
         f"segments gates={gates}")


@pytest.mark.parametrize("lens,hqk,hv", [([1500, 300], 16, 32), ([3000], 4, 8),
                                         ([900, 0, 1400, 65], 4, 8)])
def test_prefill_segments_mixed(dev, lens, hqk, hv):
    """Segmented and whole sequences in one call (short ones are not split), up to eight
    segments per sequence, empty sequences."""
    _run(dev, prefill_inputs(lens, hqk=hqk, hv=hv, seed=43, with_state=True, gates="mild",
                             state_std=0.05), f"segments lens={lens}")


@pytest.mark.parametrize("lens,plan", [
    (varlen_lengths(8, seed=7), (0, 8, 0)),  # 12, 11, 11, 8, 8, 7, 5, 2 chunks: no cut pays off
    ([4096, 700, 650], (9, 7, 0)),           # 64 chunks in 6 segments; 11-chunk ones whole in C
    ([3000, 200, 150, 100], (10, 4, 0)),     # 47 chunks in 5 segments; the short ones whole in A
    # ten sequences: pass C launched with 4 and with 8 waves. 10-12 chunks each: nothing is
    # cut, and the ten whole jobs fit the 4-wave launch
    ([720, 700, 705, 690, 680, 660, 650, 640, 600, 710], (0, 10, 0)),
    # 44-50 chunks each: all cut in 3 segments, 20 resumed segments for the 8-wave launch
    ([3000, 2900, 3100, 2950, 3050, 2800, 3200, 2850, 3150, 2990], (30, 0, 20)),
])
def test_prefill_segment_planner(dev, lens, plan):
    """Segment plans on few sequences (qk4_v8 heads; mild decay, so every chained state
    carries into the next segment). Sequences of similar length all run whole in pass C
    with pass A empty; a long sequence is cut into segments while the short ones run whole
    in pass C beside its resumed segments, or in pass A beside its segment 0 and state maps.
    Each segment kernel then runs every body it holds (whole sequence, segment with
    outputs, both state maps). The job counts the planner wrote (workspace header: pass A,
    pass C in the 4-wave launch, pass C in the 8-wave launch) name the plan taken."""
    from gdn_hip import _lib
    from gdn_hip.api import _prefill_marshal
    inp = prefill_inputs(lens, hqk=4, hv=8, seed=59, with_state=True, gates="mild",
                         state_std=0.05)
    ref_out, ref_ns = _oracle(inp)
    g = inp.to(dev)
    out = torch.empty((g.q.shape[0], 8, 128), dtype=torch.bfloat16, device=dev)
    ns = torch.empty((len(lens), 8, 128, 128), dtype=torch.float32, device=dev)
    P, _, _, copy_back, keep, stream = _prefill_marshal(*g.args(), out, ns)
    assert not copy_back
    rc = _lib.load().gdn_prefill_launch(ctypes.byref(P), ctypes.c_void_p(stream.cuda_stream))
    assert rc == 0, _lib.load().gdn_last_error()
    torch.cuda.synchronize()
    header = keep[-1][:16].view(torch.int32).cpu().tolist()
    print(f"[planner {lens[:3]}] pass A jobs {header[1]}, pass C jobs {header[2]} (4 waves) "
          f"{header[3]} (8 waves)", flush=True)
    assert (header[1], header[2], header[3]) == plan
    _check(out, ns, ref_out, ref_ns, f"planner {plan}")


@pytest.mark.parametrize("n,seed,use4", [(20, 4, True), (32, 6, False)])
def test_prefill_whole_scan_choice(dev, n, seed, use4):
    """Whole sequences with 129 to 256 (sequence, v-head) pairs: both scans are launched and
    the prep kernel gives the sequences to the 4-wave one when its load per CU stays below
    the longest sequence (20 qk4_v8 sequences), else to the 8-wave one (32 sequences). The
    workspace header holds the counts (4-wave, 8-wave); the results hold the oracle bar."""
    from gdn_hip import _lib
    from gdn_hip.api import _prefill_marshal
    lens = varlen_lengths(n, seed=seed)
    inp = prefill_inputs(lens, hqk=4, hv=8, seed=seed, with_state=True)
    ref_out, ref_ns = _oracle(inp)
    g = inp.to(dev)
    out = torch.empty((g.q.shape[0], 8, 128), dtype=torch.bfloat16, device=dev)
    ns = torch.empty((n, 8, 128, 128), dtype=torch.float32, device=dev)
    P, _, _, copy_back, keep, stream = _prefill_marshal(*g.args(), out, ns)
    assert not copy_back
    rc = _lib.load().gdn_prefill_launch(ctypes.byref(P), ctypes.c_void_p(stream.cuda_stream))
    assert rc == 0, _lib.load().gdn_last_error()
    torch.cuda.synchronize()
    header = keep[-1][:32].view(torch.int32).cpu().tolist()
    print(f"[whole scan choice N={n}] 4-wave {header[4]}, 8-wave {header[5]}", flush=True)
    assert (header[4], header[5]) == ((n, 0) if use4 else (0, n))
    _check(out, ns, ref_out, ref_ns, f"whole scan choice N={n}")


@pytest.mark.parametrize("seed", range(6))
def test_prefill_segment_planner_random(dev, seed):
    """Random mixes in the segment regime (2 to 10 sequences, qk4_v8 heads, N HV 3 <= 256):
    long sequences that may be cut beside short and empty ones, so plans mix cut sequences,
    whole jobs in either pass and the all-whole plan; mild decay keeps every chained state
    significant."""
    rng = np.random.default_rng(1000 + seed)
    n = int(rng.integers(2, 11))
    lens = [int(rng.choice([rng.integers(0, 3), rng.integers(1, 400), rng.integers(400, 1400),
                             rng.integers(1400, 3200)], p=[0.1, 0.35, 0.35, 0.2]))
            for _ in range(n)]
    _run(dev, prefill_inputs(lens, hqk=4, hv=8, seed=70 + seed, with_state=True, gates="mild",
                             state_std=0.05), f"planner mix {seed} lens={lens}")


def test_prefill_long_sequences_among_many_plan_kernel(dev):
    """Two long sequences among 68 short ones with one v-head: more than 64 sequences, so
    the plan kernel builds the tables and every sequence is scanned whole (the job planner,
    and with it segments, serves up to 64 sequences)."""
    rng = np.random.default_rng(77)
    lens = [int(x) for x in rng.integers(0, 40, 68)] + [2500, 1900]
    _run(dev, prefill_inputs(lens, hqk=1, hv=1, seed=78, with_state=True, gates="mild",
                             state_std=0.05), f"plan-kernel segments N={len(lens)}")


def test_prefill_segments_inplace_state(dev):
    """Segmented scan with new_state aliasing state: pass A reads the initial state only in
    segment 0's job, and only the last segment's pass-C job writes the final state."""
    inp = prefill_inputs([2048, 1100], seed=53, with_state=True, gates="mild", state_std=0.05)
    ref_out, ref_ns = _oracle(inp)
    g = inp.to(dev)
    out, ns = gdn_prefill(*g.args(), new_state=g.state)
    torch.cuda.synchronize()
    assert ns.data_ptr() == g.state.data_ptr()
    _check(out, ns, ref_out, ref_ns, "segments in-place")


def test_prefill_segments_match_whole_sequence_scan(dev):
    """The segmented scan and the whole-sequence scan (tuning variant 2) agree."""
    from gdn_hip.api import set_prefill_variant
    inp = prefill_inputs([1800], seed=47, with_state=True, gates="mild").to(dev)
    out_s, ns_s = gdn_prefill(*inp.args())
    try:
        set_prefill_variant(2)
        out_w, ns_w = gdn_prefill(*inp.args())
    finally:
        set_prefill_variant(0)
    torch.cuda.synchronize()
    vo = check_output(out_s, out_w.float())
    vs = check_state(ns_s, ns_w)
    print(f"[segmented vs whole] output {vo} | state {vs}", flush=True)
    assert vo.ok and vs.ok


@pytest.mark.parametrize("lens", [[300, 77, 1000], [2048]])
def test_prefill_extreme_gates(dev, lens):
    """Extreme gate inputs (softplus x > 20 branch, beta ~ 0 / ~ 1, alpha exactly 1 / 0)
    through whole-sequence and segmented scans."""
    inp = with_extreme_gates(prefill_inputs(lens, seed=63, with_state=True), seed=64)
    _run(dev, inp, f"extreme gates lens={lens}")


def _random_case(i):
    """Seeded random prefill case: sequence count and lengths (empty, sub-chunk, chunk
    multiples, long), head layout, gate regime, initial state, padding tokens, cu dtype."""
    rng = np.random.default_rng(7100 + i)
    hqk, hv = [(16, 32), (4, 8), (8, 16), (2, 8)][i % 4]
    n = int(rng.choice([1, 1, 2, 3, 4, 7, 12, 25]))
    kind = rng.choice(["empty", "short", "chunk", "medium", "long"], size=n,
                      p=[0.1, 0.2, 0.1, 0.3, 0.3])
    lens = [int({"empty": 0, "short": rng.integers(1, 64), "chunk": 64 * rng.integers(1, 6),
                 "medium": rng.integers(65, 800), "long": rng.integers(800, 3200)}[k])
            for k in kind]
    while sum(lens) > 5000:
        lens = [x // 2 for x in lens]
    gates = str(rng.choice(["strong", "mild", "none", "extreme"]))
    inp = prefill_inputs(lens, hqk=hqk, hv=hv, seed=7200 + i,
                         with_state=bool(rng.integers(0, 4) > 0),
                         gates="strong" if gates == "extreme" else gates, state_std=0.05,
                         cu_dtype=torch.int64 if rng.integers(0, 2) else torch.int32,
                         pad_tokens=int(rng.choice([0, 0, 3, 70])))
    if gates == "extreme":
        inp = with_extreme_gates(inp, seed=7300 + i)
    # segments per long sequence the launcher allows (1: whole-sequence scan)
    G = 1
    if n and n * hv * 3 <= 256:
        G = 3
        while G < 8 and n * hv * (2 * G - 1) <= 256:
            G += 1
    return inp, f"random {i}: hqk={hqk} hv={hv} gates={gates} segments<={G} lens={lens}"


@pytest.mark.parametrize("i", range(10))
def test_prefill_random_cases(dev, i):
    """Seeded random mixes that reach the planner's and the segment scan's branches
    (1..8 segments, balanced and equal segment lengths, short and empty sequences next
    to long ones) under every gate regime."""
    inp, label = _random_case(i)
    _run(dev, inp, label)


def test_prefill_long_sequence_64k(dev):
    """One 65536-token sequence (1024 chunks): eight segments of ~128 chunks with their state
    chain, mild decay so every segment's state carries into the next."""
    inp = prefill_inputs([65536], hqk=1, hv=2, seed=97, with_state=True, gates="mild",
                         state_std=0.05)
    _run(dev, inp, "1 x 65536, hqk=1 hv=2")


def test_prefill_and_decode_on_concurrent_streams(dev):
    """Two prefills in flight at once on two streams (each stream has its own cached
    workspace) and a decode on a third; every result matches the oracle."""
    from gdn_hip.inputs import decode_inputs
    ia = prefill_inputs([700, 300, 45], seed=201, with_state=True)
    ib = prefill_inputs([1500], seed=202, with_state=True, gates="mild", state_std=0.05)
    idc = decode_inputs(8, seed=203)
    ref_a, ref_b = _oracle(ia), _oracle(ib)
    ref_d = O.decode(*idc.args())
    ga, gb, gd = ia.to(dev), ib.to(dev), idc.to(dev)
    torch.cuda.synchronize()
    s1, s2, s3 = torch.cuda.Stream(dev), torch.cuda.Stream(dev), torch.cuda.Stream(dev)
    with torch.cuda.stream(s1):
        oa, na = gdn_prefill(*ga.args())
    with torch.cuda.stream(s2):
        ob, nb = gdn_prefill(*gb.args())
    with torch.cuda.stream(s3):
        od, nd = gdn_decode(*gd.args())
    torch.cuda.synchronize()
    _check(oa, na, *ref_a, "stream 1 prefill")
    _check(ob, nb, *ref_b, "stream 2 prefill")
    _check(od, nd, *ref_d, "stream 3 decode")


def test_prefill_in_graph(dev):
    """gdn_prefill captured in a HIP graph (plan, prep and scan launches): every replay, with
    eager work and a sync between replays, reproduces the eager call bit for bit."""
    inp = prefill_inputs([500, 64, 1300, 7], seed=311, with_state=True)
    ref_out, ref_ns = _oracle(inp)
    g = inp.to(dev)
    T, N = g.q.shape[0], len(inp.seqlens)
    out = torch.empty((T, 32, 128), dtype=torch.bfloat16, device=dev)
    ns = torch.empty((N, 32, 128, 128), dtype=torch.float32, device=dev)
    gdn_prefill(*g.args(), output=out, new_state=ns)
    torch.cuda.synchronize()
    _check(out, ns, ref_out, ref_ns, "eager")
    eager_out, eager_ns = out.clone(), ns.clone()
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        gdn_prefill(*g.args(), output=out, new_state=ns)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gdn_prefill(*g.args(), output=out, new_state=ns)
    for r in range(3):
        out.zero_()
        ns.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager_out), f"replay {r}: output differs"
        assert torch.equal(ns, eager_ns), f"replay {r}: new_state differs"


def test_prefill_graphs_keep_their_own_workspaces(dev):
    """Two graphs captured one after the other, the second needing a larger workspace, and
    an eager call in between: each graph keeps its own workspace, so replaying the first
    after the second (and after eager work) still reproduces its eager result bit for bit."""
    def setup(lens, seed):
        g = prefill_inputs(lens, seed=seed, with_state=True).to(dev)
        T, N = g.q.shape[0], len(lens)
        out = torch.empty((T, 32, 128), dtype=torch.bfloat16, device=dev)
        ns = torch.empty((N, 32, 128, 128), dtype=torch.float32, device=dev)
        gdn_prefill(*g.args(), output=out, new_state=ns)
        torch.cuda.synchronize()
        return g, out, ns, out.clone(), ns.clone()

    ga, oa, na, ea_o, ea_n = setup([130, 70], 401)
    gb, ob, nb, eb_o, eb_n = setup([900, 1100, 640], 402)
    graphs = []
    for g, o, n in ((ga, oa, na), (gb, ob, nb)):
        side = torch.cuda.Stream(dev)  # warm-up on a side stream, as torch.cuda.graph asks
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            gdn_prefill(*g.args(), output=o, new_state=n)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            gdn_prefill(*g.args(), output=o, new_state=n)
        graphs.append(gr)
    gdn_prefill(*gb.args())  # eager work between the replays
    for r, (gr, o, n, eo, en) in enumerate([(graphs[0], oa, na, ea_o, ea_n),
                                            (graphs[1], ob, nb, eb_o, eb_n),
                                            (graphs[0], oa, na, ea_o, ea_n)]):
        o.zero_()
        n.zero_()
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        print(f"[two graphs] replay {r} bitwise: {torch.equal(o, eo)} {torch.equal(n, en)}",
              flush=True)
        assert torch.equal(o, eo) and torch.equal(n, en), f"replay {r} differs"


def test_prefill_graph_workspaces_released_with_the_graphs(dev):
    """A captured prefill holds a workspace of its own until the caller, having destroyed the
    graph, calls release_workspace(graphs=True); the graph's replay before that matches its
    eager result, and a new capture after the release works again."""
    from gdn_hip import graph_workspace_bytes

    g = prefill_inputs([300, 41], seed=77, with_state=True).to(dev)
    T, N = g.q.shape[0], 2
    out = torch.empty((T, 32, 128), dtype=torch.bfloat16, device=dev)
    ns = torch.empty((N, 32, 128, 128), dtype=torch.float32, device=dev)
    gdn_prefill(*g.args(), output=out, new_state=ns)
    torch.cuda.synchronize()
    eo, en = out.clone(), ns.clone()
    need = _lib.load().gdn_prefill_workspace_size(T, N, 16, 32, 128)
    for rnd in range(2):
        before = graph_workspace_bytes()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            gdn_prefill(*g.args(), output=out, new_state=ns)
        assert graph_workspace_bytes() - before >= need
        out.zero_()
        ns.zero_()
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eo) and torch.equal(ns, en), f"round {rnd}: replay differs"
        del gr
        torch.cuda.synchronize()
        release_workspace(graphs=True)
        assert graph_workspace_bytes() == 0


def test_prefill_fast_path_taken_and_exact(dev):
    """A destination-passing prefill outside capture goes through the C++ fast path: it
    launches (returns 0), matches the oracle and equals the Python path bit for bit; after
    release_workspace() it allocates a fresh workspace and still matches."""
    from gdn_hip import _lib
    from gdn_hip.api import release_workspace

    fast = _lib.fast()
    assert fast is not None
    inp = prefill_inputs([300, 64, 129, 1], hqk=4, hv=8, seed=88, with_state=True)
    ref_o, ref_s = _oracle(inp)
    g = inp.to(dev)
    T, N = g.q.shape[0], len(inp.seqlens)
    out = torch.empty((T, 8, 128), dtype=torch.bfloat16, device=dev)
    ns = torch.empty((N, 8, 128, 128), dtype=torch.float32, device=dev)
    assert fast.prefill(*g.args(), out, ns, 0) == 0
    torch.cuda.synchronize()
    _check(out, ns, ref_o, ref_s, "prefill fast path")
    import ctypes

    from gdn_hip.api import _prefill_marshal
    o2, n2 = torch.empty_like(out), torch.empty_like(ns)
    P, _, _, copy_back, keep, stream = _prefill_marshal(*g.args(), o2, n2)
    assert not copy_back
    _lib.check(_lib.load().gdn_prefill_launch(ctypes.byref(P), ctypes.c_void_p(
        stream.cuda_stream)), "gdn_prefill_launch")
    torch.cuda.synchronize()
    assert torch.equal(out, o2) and torch.equal(ns, n2)
    release_workspace()
    o3, n3 = gdn_prefill(*g.args(), torch.empty_like(out), torch.empty_like(ns))
    torch.cuda.synchronize()
    assert torch.equal(out, o3) and torch.equal(ns, n3)


def test_prefill_fast_path_declines_capture_and_odd_layouts(dev):
    """Graph capture, a strided output and empty inputs go to the general path."""
    from gdn_hip import _lib

    fast = _lib.fast()
    g = prefill_inputs([70, 30], seed=89, with_state=True).to(dev)
    T = g.q.shape[0]
    out = torch.empty((T, 32, 128), dtype=torch.bfloat16, device=dev)
    ns = torch.empty((2, 32, 128, 128), dtype=torch.float32, device=dev)
    wide = torch.empty((T, 32, 256), dtype=torch.bfloat16, device=dev)
    assert fast.prefill(*g.args(), wide[..., ::2], ns, 0) == 1
    e = prefill_inputs([0, 0], seed=2, with_state=True).to(dev)
    assert fast.prefill(*e.args(), torch.empty((0, 32, 128), dtype=torch.bfloat16, device=dev),
                        torch.empty_like(e.state), 0) == 1
    fast.prefill(*g.args(), out, ns, 0)  # warm the stream's cached workspace
    torch.cuda.synchronize()
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        gdn_prefill(*g.args(), output=out, new_state=ns)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = fast.prefill(*g.args(), out, ns, 0)
    assert rc == 1
