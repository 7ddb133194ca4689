"""Randomized parity sweep of gdn_prefill and gdn_decode against the float64 CPU oracle.

Each case draws, from its own seed, a head layout (1-16 q/k heads, 1-4 v-heads per q/k
head), then for prefill a batch of 1-12 sequences whose lengths mix the chunk edges
(0, 1, 63, 64, 65, 127, 128) with random lengths up to 4000 tokens, padding tokens that
belong to no sequence, int32 or int64 cu_seqlens, a zero or random initial state and strong,
mild or no decay; for decode a batch of 1-257 sequences. Bars as in the other parity tests
(gdn_hip.parity).
"""
import random

import pytest
import torch

from gdn_hip import gdn_decode, gdn_prefill
from gdn_hip.inputs import decode_inputs, prefill_inputs
from gdn_hip.parity import check_output, check_state
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu

N_PREFILL = 32
N_DECODE = 32
SEED0 = 7000


def _layout(rnd):
    hqk = rnd.choice([1, 2, 3, 4, 8, 16])
    return hqk, hqk * rnd.choice([1, 2, 3, 4])


def _prefill_case(i):
    rnd = random.Random(SEED0 + i)
    hqk, hv = _layout(rnd)
    n = rnd.choice([1, 1, 2, 3, 5, 8, 12])
    lens = []
    for _ in range(n):
        r = rnd.random()
        if r < 0.3:
            lens.append(rnd.choice([0, 1, 63, 64, 65, 127, 128]))
        elif r < 0.9:
            lens.append(rnd.randint(1, 1500))
        else:
            lens.append(rnd.randint(1500, 4000))
    budget = max(64, 90000 // hv)  # token-heads per case: the oracle stays within seconds
    while sum(lens) > budget and max(lens) > 1:
        j = lens.index(max(lens))
        lens[j] //= 2
    return dict(hqk=hqk, hv=hv, lens=lens,
                gates=rnd.choice(["strong", "strong", "mild", "none"]),
                with_state=rnd.random() < 0.7, pad=rnd.choice([0, 0, 0, 5, 70]),
                cu=rnd.choice([torch.int32, torch.int64]))


def _decode_case(i):
    rnd = random.Random(SEED0 + 10000 + i)
    hqk, hv = _layout(rnd)
    return dict(hqk=hqk, hv=hv, batch=rnd.choice([1, 2, 3, 7, 16, 33, 64, 100, 257]),
                gates=rnd.choice(["strong", "mild", "none"]), with_state=rnd.random() < 0.8)


def _check(out, ns, ref_out, ref_ns, label):
    vo, vs = check_output(out, ref_out), check_state(ns, ref_ns)
    print(f"[{label}] output {vo} | state {vs}", flush=True)
    assert vo.ok, f"{label}: output {vo}"
    assert vs.ok, f"{label}: new_state {vs}"


@pytest.mark.parametrize("i", range(N_PREFILL))
def test_prefill_random(dev, i):
    c = _prefill_case(i)
    label = f"prefill case {i}: {c}"
    print(f"[{label}] launching", flush=True)
    inp = prefill_inputs(c["lens"], hqk=c["hqk"], hv=c["hv"], seed=SEED0 + i,
                         with_state=c["with_state"], gates=c["gates"], cu_dtype=c["cu"],
                         pad_tokens=c["pad"])
    ref_out, ref_ns = O.prefill(inp.q, inp.k, inp.v, inp.state, inp.A_log, inp.a, inp.dt_bias,
                                inp.b, inp.cu_seqlens, inp.scale)
    g = inp.to(dev)
    out, ns = gdn_prefill(*g.args())
    torch.cuda.synchronize()
    _check(out, ns, ref_out, ref_ns, label)


@pytest.mark.parametrize("i", range(N_DECODE))
def test_decode_random(dev, i):
    c = _decode_case(i)
    label = f"decode case {i}: {c}"
    print(f"[{label}] launching", flush=True)
    inp = decode_inputs(c["batch"], hqk=c["hqk"], hv=c["hv"], seed=SEED0 + 10000 + i,
                        with_state=c["with_state"], gates=c["gates"])
    ref_out, ref_ns = O.decode(inp.q, inp.k, inp.v, inp.state, inp.A_log, inp.a, inp.dt_bias,
                               inp.b, inp.scale)
    g = inp.to(dev)
    out, ns = gdn_decode(*g.args())
    torch.cuda.synchronize()
    _check(out, ns, ref_out, ref_ns, label)
