"""CPU oracle for Gated DeltaNet decode / prefill.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py``, as the result to compare against. The product (the HIP
library under ``mlsys26-flashinfer-ai-kernel-generation-contest_amd/``) never
imports this module.

Three independent restatements of the reference recurrence live here:

* ``decode`` / ``prefill``: the C oracle (``gdn_oracle.c``), token-sequential,
  float64 (parity target) or float32 (rounding-noise yardstick). Follows
  ``gdn_decode/solution/triton/kernel.py:120-131,165-170,216-218`` and the host
  contract of ``gdn_prefill/solution/triton/kernel.py:253-337``.
* ``prefill_matrix_f64``: numpy, explicit D x D matrices,
  ``S_t = alpha_t S_{t-1} (I - beta_t k_t k_t^T) + beta_t v_t k_t^T`` -- a second
  formulation of the same recurrence, for tiny brute-force cross-checks.
* ``prefill_chunked_f64``: numpy, the chunked WY/UT form
  (``gdn_prefill/solution/triton/kernel.py:60-79``; Yang et al. 2024, "Parallelizing
  Linear Transformers with the Delta Rule over Sequence Length", and "Gated Delta
  Networks") -- the algebra the HIP prefill uses, checked against the recurrence.

bf16 tensors are passed as ``uint16`` bit patterns (numpy has no bfloat16).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import threading

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_gdn.so")
_lib = None
_lock = threading.Lock()


def build(force: bool = False) -> str:
    """Compile the C oracle with gcc (via oracle/Makefile)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "-s", "-C", _HERE, "liboracle_gdn.so"],
                       check=True)
    return _LIB_PATH


def _load():
    global _lib
    with _lock:
        if _lib is None:
            build()
            lib = ctypes.CDLL(_LIB_PATH)
            P = ctypes.c_void_p
            I = ctypes.c_int
            for sfx in ("f64", "f32"):
                f = getattr(lib, f"oracle_decode_{sfx}")
                f.restype = I
                f.argtypes = [I, I, I, I, P, P, P, P, P, P, P, P, ctypes.c_double, P, P, I]
                g = getattr(lib, f"oracle_prefill_{sfx}")
                g.restype = I
                g.argtypes = [I, I, I, I, I, P, P, P, P, P, P, P, P, P, ctypes.c_double, P, P, I]
            _lib = lib
    return _lib


# ----------------------------------------------------------------------------- bf16 helpers
def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32 (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round-to-nearest-even (NaN kept quiet)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        rounded = rounded.copy()
        rounded[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return rounded


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round float values to the nearest bf16 and return them as float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(x, dtype=np.float32)))


def to_numpy(t, bf16: bool = False) -> np.ndarray:
    """Accept numpy arrays or CPU/GPU torch tensors; bf16 tensors become uint16 bits."""
    if isinstance(t, np.ndarray):
        return np.ascontiguousarray(t)
    mod = type(t).__module__
    if mod.startswith("torch"):
        import torch  # local: only when handed a tensor

        t = t.detach().to("cpu").contiguous()
        if t.dtype == torch.bfloat16:
            return t.view(torch.int16).numpy().view(np.uint16).copy()
        return t.numpy().copy()
    return np.ascontiguousarray(np.asarray(t))


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _u16(x):
    x = to_numpy(x)
    if x.dtype != np.uint16:
        raise TypeError(f"expected bf16 bits (uint16), got {x.dtype}")
    return np.ascontiguousarray(x)


def _f32(x):
    return None if x is None else np.ascontiguousarray(to_numpy(x), dtype=np.float32)


def _default_scale(scale, D):
    # gdn_decode/solution/triton/kernel.py:241-242, gdn_prefill/solution/triton/kernel.py:276-277
    if scale is None or float(scale) == 0.0:
        return 1.0 / float(np.sqrt(D))
    return float(scale)


# ----------------------------------------------------------------------------- C oracle
def decode(q, k, v, state, A_log, a, dt_bias, b, scale, precision: str = "f64", threads: int = 0):
    """Decode oracle. Shapes: q,k [B,T,HQK,D], v [B,T,HV,D], state [B,HV,D,D] or None,
    A_log/dt_bias [HV], a/b [B,T,HV]. Returns (out [B,T,HV,D], new_state [B,HV,D,D]) in
    float64 or float32 (unrounded; the reference stores out as bf16).

    T > 1: the reference launches one program per (token, value tile) and each loads the
    same input state (gdn_decode/solution/triton/kernel.py:110-118,146-147), so token t's
    output is one step from the input state; new_state is token T-1's update."""
    q, k, v, a, b = (_u16(x) for x in (q, k, v, a, b))
    A_log, dt_bias, state = _f32(A_log), _f32(dt_bias), _f32(state)
    B, T, HQK, D = q.shape
    if T < 1:
        raise ValueError("decode oracle needs seq_len >= 1")
    if T > 1:
        outs = []
        for t in range(T):
            o_t, ns = decode(q[:, t:t + 1], k[:, t:t + 1], v[:, t:t + 1], state, A_log,
                             a[:, t:t + 1], dt_bias, b[:, t:t + 1], scale, precision, threads)
            outs.append(o_t)
        return np.concatenate(outs, axis=1), ns
    HV = v.shape[2]
    scale = _default_scale(scale, D)
    dt = np.float64 if precision == "f64" else np.float32
    out = np.zeros((B, 1, HV, D), dtype=dt)
    ns = np.zeros((B, HV, D, D), dtype=dt)
    fn = getattr(_load(), f"oracle_decode_{precision}")
    rc = fn(B, HQK, HV, D, _ptr(q), _ptr(k), _ptr(v), _ptr(state), _ptr(A_log), _ptr(a),
            _ptr(dt_bias), _ptr(b), scale, _ptr(out), _ptr(ns), int(threads or os.cpu_count() or 1))
    if rc != 0:
        raise ValueError(f"oracle_decode_{precision} rejected its arguments (rc={rc})")
    return out, ns


def prefill(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, precision: str = "f64",
            threads: int = 0):
    """Prefill oracle. Shapes: q,k [T,HQK,D], v [T,HV,D], a/b [T,HV], cu_seqlens [N+1],
    state [N,HV,D,D] or None. Returns (out [T,HV,D], new_state [N,HV,D,D])."""
    q, k, v, a, b = (_u16(x) for x in (q, k, v, a, b))
    A_log, dt_bias, state = _f32(A_log), _f32(dt_bias), _f32(state)
    cu = np.ascontiguousarray(to_numpy(cu_seqlens), dtype=np.int64)
    T, HQK, D = q.shape
    HV = v.shape[1]
    N = cu.shape[0] - 1
    scale = _default_scale(scale, D)
    dt = np.float64 if precision == "f64" else np.float32
    out = np.zeros((T, HV, D), dtype=dt)
    ns = np.zeros((max(N, 0), HV, D, D), dtype=dt)
    fn = getattr(_load(), f"oracle_prefill_{precision}")
    rc = fn(T, N, HQK, HV, D, _ptr(q), _ptr(k), _ptr(v), _ptr(state), _ptr(A_log), _ptr(a),
            _ptr(dt_bias), _ptr(b), _ptr(cu), scale, _ptr(out), _ptr(ns),
            int(threads or os.cpu_count() or 1))
    if rc != 0:
        raise ValueError(f"oracle_prefill_{precision} rejected its arguments (rc={rc})")
    return out, ns


# ----------------------------------------------------------------------------- numpy restatements
def gates_f64(A_log, a, dt_bias, b):
    """alpha, beta in float64 for a/b of shape [..., HV] (bf16 bits) and A_log/dt_bias [HV].
    gdn_decode/solution/triton/kernel.py:128-131."""
    x = bf16_bits_to_f32(_u16(a)).astype(np.float64) + _f32(dt_bias).astype(np.float64)
    with np.errstate(over="ignore"):
        sp = np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))
    alpha = np.exp(-np.exp(_f32(A_log).astype(np.float64)) * sp)
    bb = bf16_bits_to_f32(_u16(b)).astype(np.float64)
    beta = 1.0 / (1.0 + np.exp(-bb))
    return alpha, beta


def prefill_matrix_f64(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale):
    """Brute force with explicit D x D transition matrices (tiny shapes only):
    S_t = alpha_t * S_{t-1} @ (I - beta_t k_t k_t^T) + beta_t v_t k_t^T,  o_t = scale * S_t q_t."""
    qf = bf16_bits_to_f32(_u16(q)).astype(np.float64)
    kf = bf16_bits_to_f32(_u16(k)).astype(np.float64)
    vf = bf16_bits_to_f32(_u16(v)).astype(np.float64)
    alpha, beta = gates_f64(A_log, a, dt_bias, b)
    cu = to_numpy(cu_seqlens).astype(np.int64)
    T, HQK, D = qf.shape
    HV = vf.shape[1]
    r = HV // HQK
    N = len(cu) - 1
    scale = _default_scale(scale, D)
    out = np.zeros((T, HV, D))
    ns = np.zeros((N, HV, D, D))
    I = np.eye(D)
    for n in range(N):
        for h in range(HV):
            g = h // r
            S = np.zeros((D, D)) if state is None else _f32(state)[n, h].astype(np.float64)
            for t in range(int(cu[n]), int(cu[n + 1])):
                kt = kf[t, g][:, None]
                M = alpha[t, h] * (I - beta[t, h] * (kt @ kt.T))
                S = S @ M + beta[t, h] * (vf[t, h][:, None] @ kt.T)
                out[t, h] = scale * (S @ qf[t, g])
            ns[n, h] = S
    return out, ns


def prefill_chunked_f64(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, chunk: int = 64):
    """Chunked WY/UT restatement in float64 (gdn_prefill/solution/triton/kernel.py:60-79).

    Per chunk with start state S0, L_t = sum_{i<=t} log alpha_i (within the chunk):
      A[t,j] = beta_t exp(L_t - L_j) (k_t . k_j),  j < t
      (I + A) U = beta * (V - exp(L) * (K S0^T))
      O = scale * (exp(L) * (Q S0^T) + (exp(L_t - L_j) (q_t . k_j))_{j<=t} U)
      S_end = exp(L_C) S0 + (exp(L_C - L_t) U_t)^T K
    Only non-positive log differences are exponentiated."""
    qf = bf16_bits_to_f32(_u16(q)).astype(np.float64)
    kf = bf16_bits_to_f32(_u16(k)).astype(np.float64)
    vf = bf16_bits_to_f32(_u16(v)).astype(np.float64)
    alpha, beta = gates_f64(A_log, a, dt_bias, b)
    with np.errstate(divide="ignore"):
        la = np.log(alpha)
    cu = to_numpy(cu_seqlens).astype(np.int64)
    T, HQK, D = qf.shape
    HV = vf.shape[1]
    r = HV // HQK
    N = len(cu) - 1
    scale = _default_scale(scale, D)
    out = np.zeros((T, HV, D))
    ns = np.zeros((N, HV, D, D))
    for n in range(N):
        s0, s1 = int(cu[n]), int(cu[n + 1])
        for h in range(HV):
            g = h // r
            S = np.zeros((D, D)) if state is None else _f32(state)[n, h].astype(np.float64)
            for c0 in range(s0, s1, chunk):
                c1 = min(c0 + chunk, s1)
                K = kf[c0:c1, g]
                Q = qf[c0:c1, g]
                V = vf[c0:c1, h]
                bt = beta[c0:c1, h]
                L = np.cumsum(la[c0:c1, h])
                diff = L[:, None] - L[None, :]
                low = np.tril(np.ones((c1 - c0, c1 - c0), dtype=bool), -1)
                incl = np.tril(np.ones((c1 - c0, c1 - c0), dtype=bool))
                dec = np.where(incl, np.exp(np.where(incl, diff, 0.0)), 0.0)
                A = np.where(low, bt[:, None] * dec * (K @ K.T), 0.0)
                R = bt[:, None] * (V - np.exp(L)[:, None] * (K @ S.T))
                U = np.linalg.solve(np.eye(c1 - c0) + A, R)
                P = dec * (Q @ K.T)
                out[c0:c1, h] = scale * (np.exp(L)[:, None] * (Q @ S.T) + P @ U)
                w = np.exp(L[-1] - L)
                S = np.exp(L[-1]) * S + (w[:, None] * U).T @ K
            ns[n, h] = S
    return out, ns
