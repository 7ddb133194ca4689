"""Write the exact known-answer fixtures for the GDN recurrence.

The reference holds no golden vectors for this path (it has no tests; its
correctness oracle lives in an external dataset), so these fixtures are computed
here in exact rational arithmetic (fractions.Fraction), independent of any
floating-point implementation. Gate inputs are chosen so the gates are exact:

* A_log = -200: exp(A_log) underflows, alpha = exp(-0 * sp) = 1 exactly
  (no decay); A_log = 10 with a + dt_bias = 1: exp(A_log) * softplus(1) ~ 2.9e4,
  alpha = exp(-2.9e4) = 0 exactly in fp32 and fp64 (full reset every token).
* b = 0: beta = sigmoid(0) = 1/2 exactly.
* q, k, v, state, scale are dyadic rationals that bf16 / fp32 hold exactly.

Recurrence (per v-head h, q/k head h // (HV/HQK), k-last state S[v][k]):
  u = alpha S k ; d = beta v + (1 - beta) u - u ; S' = alpha S + d k^T ;
  o = scale S' q                      (gdn_decode/solution/triton/kernel.py:165-170,216)

Usage: python tests/golden/make_golden.py  (writes gdn_kat_d8.npz, gdn_kat_d128.npz)
"""
from __future__ import annotations

import os
import struct
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def bf16_bits(x: float) -> int:
    """bf16 bits of a float that bf16 represents exactly (asserted)."""
    u = struct.unpack("<I", struct.pack("<f", x))[0]
    assert u & 0xFFFF == 0, f"{x} is not exactly representable in bf16"
    return u >> 16


def make(D, HQK, HV, seqlens, seed, alpha_one_heads):
    rng = np.random.default_rng(seed)
    T = sum(seqlens)
    N = len(seqlens)
    # dyadic values: multiples of 1/8 in [-1, 1] for q, k, v; 1/64 in [-1/8, 1/8] for S0
    q = rng.integers(-8, 9, size=(T, HQK, D)) / 8.0
    k = rng.integers(-8, 9, size=(T, HQK, D)) / 8.0
    v = rng.integers(-8, 9, size=(T, HV, D)) / 8.0
    s0 = rng.integers(-8, 9, size=(N, HV, D, D)) / 64.0
    A_log = np.array([-200.0 if h in alpha_one_heads else 10.0 for h in range(HV)],
                     dtype=np.float32)
    dt_bias = np.zeros(HV, dtype=np.float32)
    a = np.ones((T, HV))  # a + dt_bias = 1
    b = np.zeros((T, HV))  # beta = 1/2
    scale = 1.0 / 8.0 if D == 128 else 0.25
    alpha = {h: (Fraction(1) if h in alpha_one_heads else Fraction(0)) for h in range(HV)}
    beta = Fraction(1, 2)
    Fr = lambda x: Fraction(float(x))  # noqa: E731  (exact: all values are dyadic)
    out = np.zeros((T, HV, D))
    ns = np.zeros((N, HV, D, D))
    cu = [0]
    for L in seqlens:
        cu.append(cu[-1] + L)
    r = HV // HQK
    for n in range(N):
        for h in range(HV):
            g = h // r
            S = [[Fr(s0[n, h, i, j]) for j in range(D)] for i in range(D)]
            for t in range(cu[n], cu[n + 1]):
                kt = [Fr(x) for x in k[t, g]]
                qt = [Fr(x) for x in q[t, g]]
                al = alpha[h]
                for i in range(D):
                    row = S[i]
                    old = [al * x for x in row]
                    u = sum(o * kk for o, kk in zip(old, kt))
                    nv = beta * Fr(v[t, h, i]) + (1 - beta) * u
                    d = nv - u
                    S[i] = [o + kk * d for o, kk in zip(old, kt)]
                    out[t, h, i] = float(Fraction(scale) * sum(x * y for x, y in zip(S[i], qt)))
            for i in range(D):
                for j in range(D):
                    ns[n, h, i, j] = float(S[i][j])
    tobits = np.vectorize(bf16_bits, otypes=[np.uint16])
    return dict(
        q=tobits(q), k=tobits(k), v=tobits(v), state=s0.astype(np.float32),
        A_log=A_log, dt_bias=dt_bias, a=tobits(a), b=tobits(b),
        cu_seqlens=np.array(cu, dtype=np.int64), scale=np.float64(scale),
        out=out, new_state=ns,
    )


def main():
    d8 = make(8, 1, 2, [3, 0, 2], seed=8, alpha_one_heads={0})
    np.savez_compressed(os.path.join(HERE, "gdn_kat_d8.npz"), **d8)
    d128 = make(128, 1, 2, [3, 1], seed=128, alpha_one_heads={1})
    np.savez_compressed(os.path.join(HERE, "gdn_kat_d128.npz"), **d128)
    print("wrote gdn_kat_d8.npz, gdn_kat_d128.npz")


if __name__ == "__main__":
    main()
