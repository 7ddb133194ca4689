"""Seeded synthetic GDN workloads.

Everything is drawn on the CPU with ``torch.Generator().manual_seed(seed)`` and
then moved to the target device, so a GPU run and a CPU check see identical
bytes. Distributions:

* q, k ~ N(0, 1), L2-normalised per (token, head), then bf16; v ~ N(0, 1) bf16
* a, b ~ N(0, 1) bf16; dt_bias ~ U(-1, 1) fp32 [HV]
* A_log ~ U(0, ln 16) fp32 [HV] ("strong" gates); ``gates="mild"`` draws
  A_log ~ U(-6, -3) (alpha ~ 0.99: long memory) and ``gates="none"`` sets
  A_log = -200 (exp underflows to 0 in fp32, so alpha == 1 exactly)
* initial state ~ N(0, 0.02^2) fp32 (std 0.02), or None
* scale = 1 / sqrt(128)

The named workloads (head layout 16 q/k heads, 32 v heads, D = 128):
  decode_b1     1 sequence x 1 token (the CPU-runnable case)
  decode_b64    64 x 1 token (the HBM-bound headline)
  decode_b256   256 x 1 token, state updated in place
  prefill_4k    one 4096-token sequence, zero initial state
  prefill_16x   16 sequences, lengths ~ U[64, 1024] from the seed, non-zero state
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

HQK, HV, D = 16, 32, 128


def _gen(seed):
    g = torch.Generator()
    g.manual_seed(int(seed))
    return g


def _unit_bf16(shape, g):
    x = torch.randn(shape, generator=g, dtype=torch.float32)
    x = x / x.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    return x.to(torch.bfloat16)


def _gate_params(nv, g, gates):
    if gates == "strong":
        A_log = torch.rand(nv, generator=g) * math.log(16.0)
    elif gates == "mild":
        A_log = -6.0 + 3.0 * torch.rand(nv, generator=g)
    elif gates == "none":
        A_log = torch.full((nv,), -200.0)
    else:
        raise ValueError(f"unknown gates {gates!r}")
    dt_bias = torch.rand(nv, generator=g) * 2.0 - 1.0
    return A_log.float(), dt_bias.float()


@dataclass
class DecodeInputs:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    state: torch.Tensor | None
    A_log: torch.Tensor
    a: torch.Tensor
    dt_bias: torch.Tensor
    b: torch.Tensor
    scale: float

    def args(self):
        return (self.q, self.k, self.v, self.state, self.A_log, self.a, self.dt_bias, self.b,
                self.scale)

    def to(self, device):
        f = lambda t: None if t is None else t.to(device)  # noqa: E731
        return DecodeInputs(f(self.q), f(self.k), f(self.v), f(self.state), f(self.A_log),
                            f(self.a), f(self.dt_bias), f(self.b), self.scale)


@dataclass
class PrefillInputs:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    state: torch.Tensor | None
    A_log: torch.Tensor
    a: torch.Tensor
    dt_bias: torch.Tensor
    b: torch.Tensor
    cu_seqlens: torch.Tensor
    scale: float
    seqlens: list = field(default_factory=list)

    def args(self):
        return (self.q, self.k, self.v, self.state, self.A_log, self.a, self.dt_bias, self.b,
                self.cu_seqlens, self.scale)

    def to(self, device):
        f = lambda t: None if t is None else t.to(device)  # noqa: E731
        return PrefillInputs(f(self.q), f(self.k), f(self.v), f(self.state), f(self.A_log),
                             f(self.a), f(self.dt_bias), f(self.b), f(self.cu_seqlens),
                             self.scale, list(self.seqlens))


def with_extreme_gates(inp, seed=0):
    """Copy of ``inp`` (decode or prefill inputs) whose gate inputs take extreme values:
    a from {-30, -20.5, 19.9, 20.1, 25, 40} or N(0, 1) (both sides of softplus's x > 20
    branch), b from {-30, -8, 0, 8, 30} (beta ~ 0 .. 1), A_log per v-head from
    {-200, -10, 0, 2, 5} (alpha exactly 1 down to exactly 0)."""
    g = _gen(seed)
    a_vals = torch.tensor([-30.0, -20.5, 19.9, 20.1, 25.0, 40.0])
    b_vals = torch.tensor([-30.0, -8.0, 0.0, 8.0, 30.0])
    al_vals = torch.tensor([-200.0, -10.0, 0.0, 2.0, 5.0])
    a = inp.a.float().clone()
    pick = torch.randint(0, 8, a.shape, generator=g)
    a = torch.where(pick < 6, a_vals[pick.clamp(max=5)], a)
    b = b_vals[torch.randint(0, 5, inp.b.shape, generator=g)]
    A_log = al_vals[torch.arange(inp.A_log.shape[0]) % 5].float()
    fields = dict(inp.__dict__)
    fields.update(a=a.to(torch.bfloat16), b=b.to(torch.bfloat16), A_log=A_log)
    return type(inp)(**fields)


def decode_inputs(batch, hqk=HQK, hv=HV, d=D, seed=0, with_state=True, gates="strong",
                  state_std=0.02, seq_len=1):
    g = _gen(seed)
    q = _unit_bf16((batch, seq_len, hqk, d), g)
    k = _unit_bf16((batch, seq_len, hqk, d), g)
    v = torch.randn((batch, seq_len, hv, d), generator=g).to(torch.bfloat16)
    A_log, dt_bias = _gate_params(hv, g, gates)
    a = torch.randn((batch, seq_len, hv), generator=g).to(torch.bfloat16)
    b = torch.randn((batch, seq_len, hv), generator=g).to(torch.bfloat16)
    state = (torch.randn((batch, hv, d, d), generator=g) * state_std).float() if with_state \
        else None
    return DecodeInputs(q, k, v, state, A_log, a, dt_bias, b, 1.0 / math.sqrt(d))


def prefill_inputs(seqlens, hqk=HQK, hv=HV, d=D, seed=0, with_state=False, gates="strong",
                   state_std=0.02, cu_dtype=torch.int32, pad_tokens=0):
    """``pad_tokens`` appends tokens that belong to no sequence (output must be zero)."""
    g = _gen(seed)
    seqlens = [int(x) for x in seqlens]
    T = sum(seqlens) + int(pad_tokens)
    q = _unit_bf16((T, hqk, d), g)
    k = _unit_bf16((T, hqk, d), g)
    v = torch.randn((T, hv, d), generator=g).to(torch.bfloat16)
    A_log, dt_bias = _gate_params(hv, g, gates)
    a = torch.randn((T, hv), generator=g).to(torch.bfloat16)
    b = torch.randn((T, hv), generator=g).to(torch.bfloat16)
    cu = [0]
    for L in seqlens:
        cu.append(cu[-1] + L)
    cu_seqlens = torch.tensor(cu, dtype=cu_dtype)
    N = len(seqlens)
    state = (torch.randn((N, hv, d, d), generator=g) * state_std).float() if with_state \
        else None
    return PrefillInputs(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, 1.0 / math.sqrt(d),
                         seqlens)


def varlen_lengths(n=16, lo=64, hi=1024, seed=0):
    """Sequence lengths ~ U[lo, hi] (inclusive) drawn from the seed."""
    g = _gen(seed)
    return [int(x) for x in torch.randint(lo, hi + 1, (n,), generator=g)]


WORKLOADS = {
    "decode_b1": dict(kind="decode", batch=1),
    "decode_b64": dict(kind="decode", batch=64),
    "decode_b256": dict(kind="decode", batch=256, inplace=True),
    "prefill_4k": dict(kind="prefill", seqlens=[4096], with_state=False),
    "prefill_16x": dict(kind="prefill", seqlens=None, with_state=True),
}


def workload(name, seed=0):
    w = WORKLOADS[name]
    if w["kind"] == "decode":
        return decode_inputs(w["batch"], seed=seed)
    seqlens = w["seqlens"] or varlen_lengths(seed=seed)
    return prefill_inputs(seqlens, seed=seed, with_state=w["with_state"])


# ----------------------------------------------------------------------------- roofline bytes/flops
def decode_bytes(batch, hqk=HQK, hv=HV, d=D, with_state=True):
    """Algorithmic HBM bytes of one decode step: state read (if any) + write, q/k/v/out
    bf16, a/b bf16, A_log/dt_bias fp32."""
    state = batch * hv * d * d * 4 * (2 if with_state else 1)
    io = batch * (2 * hqk * d * 2 + 2 * hv * d * 2 + 2 * hv * 2)
    return state + io + 2 * hv * 4


def prefill_flops(tokens, hqk=HQK, hv=HV, d=D, chunk=64):
    """Canonical chunked-form FLOPs: T * [HV (6 D^2 + 6 C D) + HQK 4 C D]."""
    return tokens * (hv * (6 * d * d + 6 * chunk * d) + hqk * 4 * chunk * d)


def prefill_bytes(tokens, nseqs, hqk=HQK, hv=HV, d=D, with_state=True):
    """Algorithmic HBM bytes: q,k,v,out bf16 + a,b bf16 + state read/write fp32."""
    per_tok = 2 * hqk * d * 2 + 2 * hv * d * 2 + 2 * hv * 2
    state = nseqs * hv * d * d * 4 * (2 if with_state else 1)
    return tokens * per_tok + state + 2 * hv * 4
