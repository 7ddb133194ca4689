"""GPU parity of gdn_decode (HIP) against the float64 CPU oracle.

Bars (gdn_hip.parity): output bf16 atol = rtol = 1e-2 (both-condition rule of
FAQ.md:104-110); new_state fp32 elementwise rtol = 1e-3 / atol = 1e-4 and normwise
relative error <= 1e-3.
"""
import pytest
import torch

from gdn_hip import gdn_decode
from gdn_hip.inputs import decode_inputs, with_extreme_gates
from gdn_hip.parity import check_output, check_state
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu


def _oracle(inp):
    return O.decode(inp.q, inp.k, inp.v, inp.state, inp.A_log, inp.a, inp.dt_bias, inp.b,
                    inp.scale)


def _check(out, ns, ref_out, ref_ns, label):
    vo = check_output(out, ref_out)
    vs = check_state(ns, ref_ns)
    print(f"[{label}] output {vo} | state {vs}", flush=True)
    assert vo.ok, f"{label}: output {vo}"
    assert vs.ok, f"{label}: new_state {vs}"


@pytest.mark.parametrize("batch", [1, 7, 64, 256])
def test_decode_qk16_v32(dev, batch):
    inp = decode_inputs(batch, seed=batch)
    ref_out, ref_ns = _oracle(inp)
    g = inp.to(dev)
    inplace = batch == 256  # the in-place workload updates the state buffer itself
    out, ns = gdn_decode(*g.args(), new_state=g.state if inplace else None)
    torch.cuda.synchronize()
    if inplace:
        assert ns.data_ptr() == g.state.data_ptr()
    _check(out, ns, ref_out, ref_ns, f"B={batch}")


@pytest.mark.parametrize("batch", [1, 4, 8, 16, 32, 48, 64])
def test_decode_qk4_v8(dev, batch):
    """The contest definition gdn_decode_qk4_v8_d128_k_last over the batch sizes its
    workload set implies ({1, 4, 8, 16, 32, 48, 64})."""
    inp = decode_inputs(batch, hqk=4, hv=8, seed=100 + batch)
    ref_out, ref_ns = _oracle(inp)
    out, ns = gdn_decode(*inp.to(dev).args())
    torch.cuda.synchronize()
    _check(out, ns, ref_out, ref_ns, f"qk4_v8 B={batch}")


@pytest.mark.parametrize("hqk,hv", [(8, 8), (2, 8), (1, 4), (2, 6), (1, 7), (3, 15)])
def test_decode_head_ratios(dev, hqk, hv):
    inp = decode_inputs(5, hqk=hqk, hv=hv, seed=7)
    ref_out, ref_ns = _oracle(inp)
    out, ns = gdn_decode(*inp.to(dev).args())
    torch.cuda.synchronize()
    _check(out, ns, ref_out, ref_ns, f"hqk={hqk} hv={hv}")


@pytest.mark.parametrize("gates", ["mild", "none"])
def test_decode_gate_regimes(dev, gates):
    inp = decode_inputs(9, seed=11, gates=gates, state_std=0.5)
    ref_out, ref_ns = _oracle(inp)
    out, ns = gdn_decode(*inp.to(dev).args())
    torch.cuda.synchronize()
    _check(out, ns, ref_out, ref_ns, f"gates={gates}")


def test_decode_zero_state(dev):
    inp = decode_inputs(6, seed=3, with_state=False)
    ref_out, ref_ns = _oracle(inp)
    out, ns = gdn_decode(*inp.to(dev).args())
    torch.cuda.synchronize()
    _check(out, ns, ref_out, ref_ns, "state=None")


@pytest.mark.parametrize("scale", [None, 0.0, 0.25, "host tensor", "device tensor"])
def test_decode_scale_defaults(dev, scale):
    """scale None / 0 -> 1/sqrt(D) (gdn_decode/solution/triton/kernel.py:241-242); a
    one-element tensor is read as its value (0.25 here). Python path (no destination
    buffers) and destination-passing calls, which take the C++ fast path for a float or
    None scale and the Python path for a tensor."""
    inp = decode_inputs(3, seed=5)
    inp.scale = 0.25 if isinstance(scale, str) else scale
    ref_out, ref_ns = _oracle(inp)
    g = inp.to(dev)
    args = list(g.args())
    if isinstance(scale, str):
        args[-1] = torch.tensor([0.25], device=dev if scale == "device tensor" else "cpu")
    out, ns = gdn_decode(*args)
    o2, n2 = gdn_decode(*args, torch.empty_like(g.v), torch.empty_like(g.state))
    torch.cuda.synchronize()
    _check(out, ns, ref_out, ref_ns, f"scale={scale}")
    _check(o2, n2, ref_out, ref_ns, f"scale={scale} destination-passing")
    if not isinstance(scale, str):
        from gdn_hip import _lib

        o3, n3 = torch.empty_like(g.v), torch.empty_like(g.state)
        assert _lib.fast().decode(*args[:-1], 0.0 if scale is None else scale, o3, n3, 0) == 0
        torch.cuda.synchronize()
        assert torch.equal(o3, out) and torch.equal(n3, ns)


def test_decode_deterministic(dev):
    inp = decode_inputs(64, seed=9).to(dev)
    o1, s1 = gdn_decode(*inp.args())
    o2, s2 = gdn_decode(*inp.args())
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)


def test_decode_strided_views_and_canaries(dev):
    """Non-contiguous inputs/outputs; writes stay inside the views."""
    B, HQK, HV, D = 4, 16, 32, 128
    inp = decode_inputs(B, seed=13)
    ref_out, ref_ns = _oracle(inp)
    g = inp.to(dev)
    # q/k/v as views into wider buffers (head-interleaved, as a fused qkv projection gives)
    qkv = torch.zeros((B, 1, 2 * HQK + HV, D), dtype=torch.bfloat16, device=dev)
    qkv[:, :, :HQK] = g.q
    qkv[:, :, HQK:2 * HQK] = g.k
    qkv[:, :, 2 * HQK:] = g.v
    q, k, v = qkv[:, :, :HQK], qkv[:, :, HQK:2 * HQK], qkv[:, :, 2 * HQK:]
    # transposed (non-unit inner stride) a: forces the wrapper's contiguous copy path
    a_t = g.a.transpose(0, 2).contiguous().transpose(0, 2)
    poison = -12345.0
    big_ns = torch.full((B, HV + 2, D, D), poison, dtype=torch.float32, device=dev)
    ns_view = big_ns[:, 1:HV + 1]
    big_out = torch.full((B, 1, HV + 3, D), poison, dtype=torch.bfloat16, device=dev)
    out_view = big_out[:, :, 2:HV + 2]
    out, ns = gdn_decode(q, k, v, g.state, g.A_log, a_t, g.dt_bias, g.b, g.scale,
                         output=out_view, new_state=ns_view)
    torch.cuda.synchronize()
    assert out.data_ptr() == out_view.data_ptr() and ns.data_ptr() == ns_view.data_ptr()
    _check(out, ns, ref_out, ref_ns, "strided")
    assert torch.all(big_ns[:, 0] == poison) and torch.all(big_ns[:, HV + 1] == poison)
    assert torch.all(big_out[:, :, :2] == poison) and torch.all(big_out[:, :, HV + 2:] == poison)


def test_decode_batch_zero(dev):
    inp = decode_inputs(0, seed=1).to(dev)
    out, ns = gdn_decode(*inp.args())
    assert out.shape == (0, 1, 32, 128) and ns.shape == (0, 32, 128, 128)


def test_decode_loaded_native_library():
    """The process loaded the in-tree libgdn_hip.so and one HIP runtime."""
    maps = open("/proc/self/maps").read()
    assert "libgdn_hip.so" in maps
    hip = {ln.split()[-1] for ln in maps.splitlines() if "libamdhip64" in ln}
    assert len(hip) == 1, hip


def test_decode_matches_exact_fixture(dev):
    """HIP decode of the fixture's single-token sequence vs its rational known answer."""
    import os

    import numpy as np

    f = np.load(os.path.join(os.path.dirname(__file__), "golden", "gdn_kat_d128.npz"))
    t = int(f["cu_seqlens"][1])  # second sequence: exactly one token

    def bf(x):
        return torch.from_numpy(np.ascontiguousarray(x).view(np.int16).copy()).view(
            torch.bfloat16).to(dev)

    out, ns = gdn_decode(bf(f["q"][t:t + 1][None]), bf(f["k"][t:t + 1][None]),
                         bf(f["v"][t:t + 1][None]), torch.from_numpy(f["state"][1:2]).to(dev),
                         torch.from_numpy(f["A_log"]).to(dev), bf(f["a"][t:t + 1][None]),
                         torch.from_numpy(f["dt_bias"]).to(dev), bf(f["b"][t:t + 1][None]),
                         float(f["scale"]))
    torch.cuda.synchronize()
    _check(out[0, 0], ns[0], f["out"][t], f["new_state"][1], "exact fixture")


@pytest.mark.parametrize("batch,seq_len", [(3, 2), (5, 4), (64, 3)])
def test_decode_multi_token(dev, batch, seq_len):
    """seq_len > 1: every token is one step from the input state; new_state is the last
    token's update (gdn_decode/solution/triton/kernel.py:110-118,146-147)."""
    inp = decode_inputs(batch, seed=40 + seq_len, seq_len=seq_len)
    ref_out, ref_ns = _oracle(inp)
    g = inp.to(dev)
    out, ns = gdn_decode(*g.args())
    torch.cuda.synchronize()
    assert out.shape == (batch, seq_len, 32, 128)
    _check(out, ns, ref_out, ref_ns, f"B={batch} T={seq_len}")
    # the last token alone gives the same bits
    last = decode_inputs(batch, seed=40 + seq_len, seq_len=seq_len)
    for f in ("q", "k", "v", "a", "b"):
        setattr(last, f, getattr(last, f)[:, -1:])
    o1, s1 = gdn_decode(*last.to(dev).args())
    torch.cuda.synchronize()
    assert torch.equal(o1[:, 0], out[:, -1]) and torch.equal(s1, ns)


def test_decode_multi_token_in_place_and_strided(dev):
    """seq_len > 1 with new_state = state (the wrapper reads a copy) and token-strided
    views of a wider q/k/v buffer."""
    B, T, HQK, HV, D = 4, 3, 16, 32, 128
    inp = decode_inputs(B, seed=77, seq_len=T)
    ref_out, ref_ns = _oracle(inp)
    g = inp.to(dev)
    qkv = torch.zeros((B, T, 2 * HQK + HV, D), dtype=torch.bfloat16, device=dev)
    qkv[:, :, :HQK] = g.q
    qkv[:, :, HQK:2 * HQK] = g.k
    qkv[:, :, 2 * HQK:] = g.v
    q, k, v = qkv[:, :, :HQK], qkv[:, :, HQK:2 * HQK], qkv[:, :, 2 * HQK:]
    out, ns = gdn_decode(q, k, v, g.state, g.A_log, g.a, g.dt_bias, g.b, g.scale,
                         new_state=g.state)
    torch.cuda.synchronize()
    assert ns.data_ptr() == g.state.data_ptr()
    _check(out, ns, ref_out, ref_ns, "T=3 in place, strided")


@pytest.mark.parametrize("seq_len", [1, 3])
def test_decode_extreme_gates(dev, seq_len):
    """Gate inputs on both sides of softplus's x > 20 branch, beta ~ 0 and ~ 1, alpha
    exactly 1 and exactly 0 (kernel.py:128-131)."""
    inp = with_extreme_gates(decode_inputs(16, seed=61, seq_len=seq_len), seed=62)
    ref_out, ref_ns = _oracle(inp)
    g = inp.to(dev)
    out, ns = gdn_decode(*g.args())
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all() and torch.isfinite(ns).all()
    _check(out, ns, ref_out, ref_ns, f"extreme gates T={seq_len}")


def test_decode_state_offsets_beyond_32_bits(dev):
    """A state view whose batch stride is 2^31 elements takes the kernel's 64-bit offset
    instantiation (every other test fits 32-bit offsets)."""
    inp = decode_inputs(2, seed=77)
    ref_out, ref_ns = _oracle(inp)
    g = inp.to(dev)
    n = 32 * 128 * 128
    big = torch.empty((1 << 31) + n, dtype=torch.float32, device=dev)  # 8 GiB
    try:
        st = big.as_strided((2, 32, 128, 128), (1 << 31, 128 * 128, 128, 1))
        st.copy_(g.state)
        out, ns = gdn_decode(g.q, g.k, g.v, st, g.A_log, g.a, g.dt_bias, g.b, g.scale)
        torch.cuda.synchronize()
        _check(out, ns, ref_out, ref_ns, "state batch stride 2^31")
        inpl_out, inpl_ns = gdn_decode(g.q, g.k, g.v, st, g.A_log, g.a, g.dt_bias, g.b, g.scale,
                                       new_state=st)
        torch.cuda.synchronize()
        assert inpl_ns.data_ptr() == st.data_ptr()
        _check(inpl_out, st.clone(), ref_out, ref_ns, "state batch stride 2^31, in place")
    finally:
        del big
        torch.cuda.empty_cache()


def test_decode_more_sequences_than_one_grid(dev):
    """B above 65535 is launched in slices of at most 65535 sequences (a grid dimension);
    sequences on both sides of the slice boundary match the oracle."""
    B = 65537
    inp = decode_inputs(B, hqk=1, hv=1, seed=91)  # one head: 4 GiB of fp32 state
    g = inp.to(dev)
    out, ns = gdn_decode(*g.args())
    torch.cuda.synchronize()
    idx = torch.tensor([0, 1, 65533, 65534, 65535, 65536])
    sub = type(inp)(inp.q[idx], inp.k[idx], inp.v[idx], inp.state[idx], inp.A_log, inp.a[idx],
                    inp.dt_bias, inp.b[idx], inp.scale)
    ref_out, ref_ns = _oracle(sub)
    di = idx.to(dev)
    _check(out[di], ns[di], ref_out, ref_ns, f"B={B}, sequences {idx.tolist()}")
    del g, out, ns
    torch.cuda.empty_cache()


def test_decode_plan_in_graph(dev):
    """A DecodePlan step captured in a HIP graph: every replay, with eager work and a sync
    between replays, reproduces the eager launch bit for bit."""
    from gdn_hip.api import DecodePlan
    inp = decode_inputs(16, seed=301)
    ref_out, ref_ns = _oracle(inp)
    g = inp.to(dev)
    out, ns = torch.empty_like(g.v), torch.empty_like(g.state)
    plan = DecodePlan(g.q, g.k, g.v, g.state, g.A_log, g.a, g.dt_bias, g.b, g.scale, out, ns)
    plan.run()
    torch.cuda.synchronize()
    _check(out, ns, ref_out, ref_ns, "eager")
    eager_out, eager_ns = out.clone(), ns.clone()
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        plan.run()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.run()
    for r in range(3):
        out.zero_()
        ns.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager_out), f"replay {r}: output differs"
        assert torch.equal(ns, eager_ns), f"replay {r}: new_state differs"


def test_decode_fast_path_taken_and_exact(dev):
    """A destination-passing call with in-place-usable buffers goes through the C++ fast
    path (validation and marshalling in C++): it launches (returns 0), matches the oracle
    and equals the Python path's result bit for bit."""
    from gdn_hip import _lib
    from gdn_hip.api import _decode_marshal

    fast = _lib.fast()
    assert fast is not None, "fast-path extension not built (gdn_hip.build.build_fast)"
    inp = decode_inputs(16, hqk=4, hv=8, seed=77)
    ref_out, ref_ns = _oracle(inp)
    g = inp.to(dev)
    out, ns = torch.empty_like(g.v), torch.empty_like(g.state)
    assert fast.decode(*g.args(), out, ns, 0) == 0
    torch.cuda.synchronize()
    _check(out, ns, ref_out, ref_ns, "fast path")
    # the Python path (ctypes) on the same inputs
    P, o2, n2, copy_back, keep = _decode_marshal(*g.args(), torch.empty_like(out),
                                                 torch.empty_like(ns))
    import ctypes
    _lib.check(_lib.load().gdn_decode_launch(ctypes.byref(P), ctypes.c_void_p(
        torch.cuda.current_stream(dev).cuda_stream)), "gdn_decode_launch")
    torch.cuda.synchronize()
    assert torch.equal(out, o2) and torch.equal(ns, n2)


def test_decode_fast_path_declines_what_it_cannot_use(dev):
    """Calls the fast path cannot serve in place return 1 (the general path then handles
    them): a non-unit inner stride, a CPU tensor, a wrong dtype, mismatched shapes and an
    in-place state with a token axis. The public entry point still serves the strided
    output correctly."""
    from gdn_hip import _lib

    fast = _lib.fast()
    inp = decode_inputs(4, seed=5)
    g = inp.to(dev)
    out, ns = torch.empty_like(g.v), torch.empty_like(g.state)
    a = list(g.args())
    wide = torch.empty((4, 1, 32, 256), dtype=torch.bfloat16, device=dev)
    assert fast.decode(*a, wide[..., ::2], ns, 0) == 1
    a_cpu = list(a)
    a_cpu[0] = a[0].cpu()
    assert fast.decode(*a_cpu, out, ns, 0) == 1
    a_dt = list(a)
    a_dt[4] = a[4].double()
    assert fast.decode(*a_dt, out, ns, 0) == 1
    assert fast.decode(*a, out, ns[:2], 0) == 1
    t2 = decode_inputs(3, seed=6, seq_len=2).to(dev)
    st = t2.state.clone()
    args2 = list(t2.args())
    args2[3] = st
    assert fast.decode(*args2, torch.empty_like(t2.v), st, 0) == 1
    ref_out, ref_ns = _oracle(inp)
    o, s = gdn_decode(*g.args(), wide[..., ::2], ns)
    torch.cuda.synchronize()
    _check(o, s, ref_out, ref_ns, "general path via strided output")


def test_stale_hip_error_is_reported_not_blamed(dev):
    """A HIP error an earlier call left pending (here hipSetDevice on a device that does
    not exist) does not fail the next decode: it launches, matches the oracle, returns
    GDN_OK, and its last-error message names the drained error."""
    import ctypes

    from gdn_hip import _lib

    lib = _lib.load()
    path = next(ln.split()[-1] for ln in open("/proc/self/maps").read().splitlines()
                if "libamdhip64" in ln)
    hip = ctypes.CDLL(path)
    inp = decode_inputs(2, seed=12)
    ref_out, ref_ns = _oracle(inp)
    g = inp.to(dev)
    from gdn_hip.api import _decode_marshal

    P, out, ns, copy_back, keep = _decode_marshal(*g.args(), torch.empty_like(g.v),
                                                  torch.empty_like(g.state))
    torch.cuda.synchronize()
    assert hip.hipSetDevice(ctypes.c_int(4096)) != 0  # leaves hipErrorInvalidDevice pending
    rc = lib.gdn_decode_launch(ctypes.byref(P), ctypes.c_void_p(
        torch.cuda.current_stream(dev).cuda_stream))
    msg = _lib.last_error()
    torch.cuda.synchronize()
    print(f"rc={rc} last_error={msg!r}", flush=True)
    assert rc == _lib.GDN_OK
    assert msg.startswith("note:") and "Invalid" in msg, msg
    _check(out, ns, ref_out, ref_ns, "after a stale HIP error")

