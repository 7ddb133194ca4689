"""CPU tests pinning the oracle (oracle/gdn_oracle.*) before results are compared against it.

The reference ships no golden vectors for this path, so the oracle is pinned by:
* exact known answers (tests/golden/*.npz, computed in rational arithmetic by
  tests/golden/make_golden.py with gates that are exactly 0, 1 or 1/2);
* the gate formulas checked against Python's math library, including the
  softplus threshold (gdn_decode/solution/triton/kernel.py:128-131);
* an independent formulation (explicit D x D transition matrices) and the chunked
  WY/UT algebra (C in {1, 3, 16, 64}) agreeing with the token recurrence;
* invariants: prefill of single tokens == decode, resume split, linearity in v,
  GVA head permutation, varlen packing / order independence, empty sequences,
  beta = 0, alpha = 0 reset, and the no-decay closed form.
Each check is built so that a plausible slip (transposed state, wrong GVA map,
readout before the update, dropped decay, wrong sign in the delta rule) fails it.
"""
import math
import os

import numpy as np
import pytest

from oracle import gdn_oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _bf(x):
    return O.f32_to_bf16_bits(np.asarray(x, dtype=np.float32))


def _rand_case(rng, T, HQK, HV, D, N_lens, with_state=True, alog=(0.0, math.log(16.0))):
    q = rng.standard_normal((T, HQK, D))
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k = rng.standard_normal((T, HQK, D))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((T, HV, D))
    a = rng.standard_normal((T, HV))
    b = rng.standard_normal((T, HV))
    A_log = rng.uniform(*alog, HV).astype(np.float32)
    dt = rng.uniform(-1, 1, HV).astype(np.float32)
    cu = np.concatenate([[0], np.cumsum(N_lens)]).astype(np.int64)
    st = (rng.standard_normal((len(N_lens), HV, D, D)) * 0.1).astype(np.float32) if with_state \
        else None
    return dict(q=_bf(q), k=_bf(k), v=_bf(v), state=st, A_log=A_log, a=_bf(a), dt_bias=dt,
                b=_bf(b), cu_seqlens=cu, scale=1.0 / math.sqrt(D))


def _prefill(c, fn=O.prefill, **kw):
    return fn(c["q"], c["k"], c["v"], c["state"], c["A_log"], c["a"], c["dt_bias"], c["b"],
              c["cu_seqlens"], c["scale"], **kw)


# ----------------------------------------------------------------------------- exact fixtures
@pytest.mark.parametrize("name", ["gdn_kat_d8.npz", "gdn_kat_d128.npz"])
def test_oracle_matches_exact_fixture(name):
    f = np.load(os.path.join(GOLDEN, name))
    out, ns = O.prefill(f["q"], f["k"], f["v"], f["state"], f["A_log"], f["a"], f["dt_bias"],
                        f["b"], f["cu_seqlens"], float(f["scale"]))
    np.testing.assert_allclose(out, f["out"], rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(ns, f["new_state"], rtol=1e-12, atol=1e-13)


def test_fixture_is_not_trivially_satisfied():
    """A transposed state or a readout before the update must miss the fixture."""
    f = np.load(os.path.join(GOLDEN, "gdn_kat_d8.npz"))
    st_t = np.ascontiguousarray(np.swapaxes(f["state"], -1, -2))
    out, ns = O.prefill(f["q"], f["k"], f["v"], st_t, f["A_log"], f["a"], f["dt_bias"], f["b"],
                        f["cu_seqlens"], float(f["scale"]))
    assert np.abs(ns - f["new_state"]).max() > 1e-3
    # readout with the pre-update state: o = scale * S_{t-1} q_t differs from the fixture
    q = O.bf16_bits_to_f32(f["q"]).astype(np.float64)
    s0 = f["state"].astype(np.float64)
    pre = float(f["scale"]) * s0[0, 0] @ q[0, 0]
    assert np.abs(pre - f["out"][0, 0]).max() > 1e-3


# ----------------------------------------------------------------------------- gates
@pytest.mark.parametrize("A_log,a,dt,b", [
    (0.0, 0.0, 0.0, 0.0), (math.log(16.0), 1.5, -0.25, -2.0), (1.0, -3.0, 0.5, 3.0),
    (0.5, 19.5, 0.25, 0.5),   # x = 19.75: log(1 + e^x) branch
    (0.25, 22.0, 1.0, -1.0),  # x = 23 > 20: softplus(x) = x exactly
    (-4.0, -30.0, 0.0, 8.0),
])
def test_gates_against_math_library(A_log, a, dt, b):
    """alpha and beta recovered from the oracle's state update match math.exp/log1p.

    With k = 0 the update is S' = alpha S (u = 0, delta = beta v k^T = 0); with S = 0
    and a unit k it is S' = beta v k^T."""
    D, HV = 4, 1
    ab = _bf([[[a]]])
    bb = _bf([[[b]]])
    # the bf16 rounding of a and b is part of the input contract
    a_r = float(O.bf16_bits_to_f32(ab).ravel()[0])
    b_r = float(O.bf16_bits_to_f32(bb).ravel()[0])
    x = a_r + float(np.float32(dt))
    sp = x if x > 20.0 else math.log1p(math.exp(x))
    alpha = math.exp(-math.exp(float(np.float32(A_log))) * sp)
    beta = 1.0 / (1.0 + math.exp(-b_r))
    zeros = _bf(np.zeros((1, 1, 1, D)))
    e0 = _bf(np.eye(D)[0][None, None, None, :])
    v = _bf(np.array([0.5, -1.0, 0.25, 2.0])[None, None, None, :])
    S0 = np.eye(D, dtype=np.float32)[None, None]
    args = (np.float32([A_log]), ab, np.float32([dt]), bb, 1.0)
    _, ns = O.decode(zeros, zeros, v, S0, args[0], args[1], args[2], args[3], args[4])
    np.testing.assert_allclose(ns[0, 0], alpha * np.eye(D), rtol=1e-13, atol=1e-300)
    _, ns = O.decode(zeros, e0, v, None, args[0], args[1], args[2], args[3], args[4])
    expect = beta * np.outer(O.bf16_bits_to_f32(v).ravel(), np.eye(D)[0])
    np.testing.assert_allclose(ns[0, 0], expect, rtol=1e-13, atol=1e-300)


# ----------------------------------------------------------------------------- formulations
@pytest.mark.parametrize("HQK,HV,D,lens", [
    (1, 1, 4, [5]), (1, 2, 8, [3, 0, 4]), (2, 4, 8, [7, 1]), (2, 8, 16, [9]),
    (4, 8, 32, [6, 2, 3]),
])
def test_c_oracle_equals_matrix_form(HQK, HV, D, lens):
    c = _rand_case(np.random.default_rng(D * 10 + HV), sum(lens), HQK, HV, D, lens)
    o1, s1 = _prefill(c)
    o2, s2 = _prefill(c, fn=O.prefill_matrix_f64)
    np.testing.assert_allclose(o1, o2, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(s1, s2, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("chunk", [1, 3, 16, 64])
@pytest.mark.parametrize("alog", [(0.0, math.log(16.0)), (-6.0, -3.0)])
def test_chunked_wy_form_equals_recurrence(chunk, alog):
    c = _rand_case(np.random.default_rng(chunk), 150, 2, 4, 16, [70, 0, 80], alog=alog)
    o1, s1 = _prefill(c)
    o2, s2 = _prefill(c, fn=O.prefill_chunked_f64, chunk=chunk)
    np.testing.assert_allclose(o1, o2, rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(s1, s2, rtol=1e-9, atol=1e-11)


def test_f32_oracle_close_to_f64():
    c = _rand_case(np.random.default_rng(3), 300, 2, 4, 128, [200, 100])
    o1, s1 = _prefill(c)
    o2, s2 = _prefill(c, precision="f32")
    assert np.abs(s1 - s2).max() < 1e-5 * max(1.0, np.abs(s1).max())
    assert np.abs(o1 - o2).max() < 1e-5 * max(1.0, np.abs(o1).max())


# ----------------------------------------------------------------------------- invariants
def test_prefill_single_tokens_equal_decode():
    rng = np.random.default_rng(5)
    B, HQK, HV, D = 6, 2, 4, 16
    c = _rand_case(rng, B, HQK, HV, D, [1] * B)
    o1, s1 = _prefill(c)
    o2, s2 = O.decode(c["q"][:, None], c["k"][:, None], c["v"][:, None], c["state"], c["A_log"],
                      c["a"][:, None], c["dt_bias"], c["b"][:, None], c["scale"])
    np.testing.assert_array_equal(o1, o2[:, 0])
    np.testing.assert_array_equal(s1, s2)


def test_resume_split():
    c = _rand_case(np.random.default_rng(6), 50, 1, 2, 8, [50], alog=(-5.0, -2.0))
    o, s = _prefill(c)
    m = 17
    c1 = dict(c, q=c["q"][:m], k=c["k"][:m], v=c["v"][:m], a=c["a"][:m], b=c["b"][:m],
              cu_seqlens=np.array([0, m]))
    o1, s1 = _prefill(c1)
    c2 = dict(c, q=c["q"][m:], k=c["k"][m:], v=c["v"][m:], a=c["a"][m:], b=c["b"][m:],
              cu_seqlens=np.array([0, 50 - m]), state=s1.astype(np.float32))
    o2, s2 = _prefill(c2)
    # the state handed over is rounded to fp32 (the caller's dtype)
    np.testing.assert_allclose(np.concatenate([o1, o2]), o, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(s2, s, rtol=1e-6, atol=1e-7)


def test_linear_in_v_with_zero_state():
    rng = np.random.default_rng(7)
    c = _rand_case(rng, 20, 1, 2, 8, [20], with_state=False)
    v1 = rng.integers(-4, 5, size=(20, 2, 8)) / 4.0
    v2 = rng.integers(-4, 5, size=(20, 2, 8)) / 4.0
    outs = []
    for vv in (v1, v2, v1 + v2):  # all exact in bf16
        o, s = _prefill(dict(c, v=_bf(vv)))
        outs.append((o, s))
    np.testing.assert_allclose(outs[0][0] + outs[1][0], outs[2][0], rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(outs[0][1] + outs[1][1], outs[2][1], rtol=1e-10, atol=1e-12)


def test_gva_head_permutation():
    """Swapping q/k heads 0 and 1 swaps the v-head pairs {0,1} and {2,3}."""
    c = _rand_case(np.random.default_rng(8), 12, 2, 4, 8, [12])
    o, s = _prefill(c)
    pq = [1, 0]
    pv = [2, 3, 0, 1]
    c2 = dict(c, q=c["q"][:, pq], k=c["k"][:, pq], v=c["v"][:, pv], a=c["a"][:, pv],
              b=c["b"][:, pv], A_log=c["A_log"][pv], dt_bias=c["dt_bias"][pv],
              state=np.ascontiguousarray(c["state"][:, pv]))
    o2, s2 = _prefill(c2)
    np.testing.assert_array_equal(o2, o[:, pv])
    np.testing.assert_array_equal(s2, s[:, pv])


def test_varlen_packing_is_independent_per_sequence():
    rng = np.random.default_rng(9)
    lens = [5, 0, 9, 3]
    c = _rand_case(rng, sum(lens), 1, 2, 8, lens)
    o, s = _prefill(c)
    cu = c["cu_seqlens"]
    for n, L in enumerate(lens):
        sl = slice(int(cu[n]), int(cu[n + 1]))
        cn = dict(c, q=c["q"][sl], k=c["k"][sl], v=c["v"][sl], a=c["a"][sl], b=c["b"][sl],
                  cu_seqlens=np.array([0, L]), state=c["state"][n:n + 1])
        on, sn = _prefill(cn)
        np.testing.assert_array_equal(on, o[sl])
        np.testing.assert_array_equal(sn[0], s[n])


def test_empty_inputs_keep_state_and_zero_output():
    c = _rand_case(np.random.default_rng(10), 7, 1, 2, 8, [0, 0])
    # tokens exist but belong to no sequence: output zero, states unchanged
    o, s = _prefill(dict(c, cu_seqlens=np.array([0, 0, 0])))
    assert np.all(o == 0)
    np.testing.assert_array_equal(s, c["state"].astype(np.float64))


def test_beta_zero_only_decays():
    c = _rand_case(np.random.default_rng(11), 4, 1, 2, 8, [4])
    c["b"] = _bf(np.full((4, 2), -200.0))  # sigmoid(-200) ~ 1e-87
    o, s = _prefill(c)
    alpha, _ = O.gates_f64(c["A_log"], c["a"], c["dt_bias"], c["b"])
    expect = c["state"][0].astype(np.float64) * np.prod(alpha, axis=0)[:, None, None]
    np.testing.assert_allclose(s[0], expect, rtol=1e-12, atol=1e-80)


def test_alpha_zero_resets_to_last_outer_product():
    """Strong decay (alpha underflows to 0): S' = beta v k^T of the last token only."""
    c = _rand_case(np.random.default_rng(12), 5, 1, 2, 8, [5])
    c["A_log"] = np.float32([10.0, 10.0])
    c["a"] = _bf(np.full((5, 2), 5.0))
    o, s = _prefill(c)
    _, beta = O.gates_f64(c["A_log"], c["a"], c["dt_bias"], c["b"])
    k = O.bf16_bits_to_f32(c["k"]).astype(np.float64)
    v = O.bf16_bits_to_f32(c["v"]).astype(np.float64)
    for h in range(2):
        np.testing.assert_allclose(s[0, h], beta[-1, h] * np.outer(v[-1, h], k[-1, 0]),
                                   rtol=1e-14, atol=1e-15)


def test_no_decay_single_token_closed_form():
    """alpha = 1, beta = 1, S0 = 0, unit k: S' = v k^T and o = scale (k . q) v."""
    D = 8
    rng = np.random.default_rng(13)
    k = np.zeros(D)
    k[3] = 1.0
    q = rng.integers(-4, 5, size=D) / 4.0
    v = rng.integers(-4, 5, size=D) / 4.0
    c = dict(q=_bf(q[None, None]), k=_bf(k[None, None]), v=_bf(v[None, None]), state=None,
             A_log=np.float32([-200.0]), a=_bf([[0.0]]), dt_bias=np.float32([0.0]),
             b=_bf([[200.0]]), cu_seqlens=np.array([0, 1]), scale=0.5)
    o, s = _prefill(c)
    np.testing.assert_allclose(s[0, 0], np.outer(v, k), rtol=0, atol=1e-15)
    np.testing.assert_allclose(o[0, 0], 0.5 * (k @ q) * v, rtol=0, atol=1e-15)


def test_oracle_rejects_bad_cu_seqlens():
    c = _rand_case(np.random.default_rng(14), 6, 1, 1, 4, [6])
    with pytest.raises(ValueError):
        _prefill(dict(c, cu_seqlens=np.array([0, 7])))
    with pytest.raises(ValueError):
        _prefill(dict(c, cu_seqlens=np.array([3, 2])))
