"""Correctness rule and error statistics.

The contest rule (FAQ.md:104-110): an element fails only if BOTH
``|x - ref| > atol`` AND ``|x - ref| > rtol * |ref|``; a workload passes when the
matched fraction reaches ``required_matched_ratio`` (1.0 for GDN). A failing
workload zeroes the kernel's score (computer_track_scores_local.py:157-158).

Bars used for this path (every test, the harness and smoke()):
* output (bf16):    atol = rtol = 1e-2, the contest's GDN tolerance (FAQ.md:104-110);
                    tighter than the 2e-2 the benchmark specification allows.
* new_state (fp32): elementwise atol = 1e-4, rtol = 1e-3 (both-condition rule), AND the
                    normwise relative error ||x - ref|| / ||ref|| <= 1e-3 ("1e-3 relative
                    on fp32 new_state"). The contest itself holds new_state to 1e-2.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

# gdn (DSA / GDN) row of FAQ.md:104-110
CONTEST_TOL = dict(atol=1e-2, rtol=1e-2)
OUT_TOL = dict(CONTEST_TOL)
STATE_TOL = dict(atol=1e-4, rtol=1e-3)
STATE_NORM_RTOL = 1e-3


@dataclass
class Verdict:
    ok: bool
    max_abs: float
    max_rel: float
    n_fail: int
    n: int
    norm_rel: float
    norm_bar: float | None = None  # normwise bar applied (None: elementwise only)

    def __str__(self):
        bar = "" if self.norm_bar is None else f" (<= {self.norm_bar:g})"
        return (f"{'PASSED' if self.ok else 'FAILED'} max_abs={self.max_abs:.3e} "
                f"max_rel={self.max_rel:.3e} norm_rel={self.norm_rel:.3e}{bar} "
                f"fail={self.n_fail}/{self.n}")


def _np(x):
    if isinstance(x, np.ndarray):
        return x.astype(np.float64)
    mod = type(x).__module__
    if mod.startswith("torch"):
        return x.detach().float().cpu().numpy().astype(np.float64)
    return np.asarray(x, dtype=np.float64)


def compare(actual, expected, atol, rtol, required_matched_ratio=1.0,
            norm_rtol=None) -> Verdict:
    """Both-condition elementwise rule; with ``norm_rtol`` the normwise relative error
    must also stay within it (an all-zero reference then needs an all-zero result)."""
    a, e = _np(actual), _np(expected)
    if a.shape != e.shape:
        raise ValueError(f"shape mismatch {a.shape} vs {e.shape}")
    d = np.abs(a - e)
    finite = np.isfinite(a)
    with np.errstate(divide="ignore", invalid="ignore"):
        rel = np.where(e != 0, d / np.abs(e), np.where(d == 0, 0.0, np.inf))
    fail = (~finite) | ((d > atol) & (d > rtol * np.abs(e)))
    n = a.size
    nf = int(fail.sum())
    ok = n == 0 or (1.0 - nf / n) >= required_matched_ratio
    en = float(np.linalg.norm(e))
    dn = float(np.linalg.norm(np.where(finite, a - e, np.inf)))
    norm_rel = dn / en if en > 0 else dn
    if norm_rtol is not None and n:
        ok = ok and (norm_rel <= norm_rtol if en > 0 else dn == 0.0)
    return Verdict(ok=ok, max_abs=float(d.max()) if n else 0.0,
                   max_rel=float(rel[np.isfinite(rel)].max()) if n and np.isfinite(rel).any()
                   else 0.0, n_fail=nf, n=n, norm_rel=norm_rel, norm_bar=norm_rtol)


def check_output(actual, expected) -> Verdict:
    return compare(actual, expected, **OUT_TOL)


def check_state(actual, expected) -> Verdict:
    return compare(actual, expected, **STATE_TOL, norm_rtol=STATE_NORM_RTOL)
