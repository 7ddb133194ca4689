"""CPU tests of the host wrappers' argument handling: every malformed call raises
TypeError / ValueError before any kernel launch, and nothing falls back to a CPU
computation (gdn_decode/solution/triton/kernel.py:221-272,
gdn_prefill/solution/triton/kernel.py:253-337 define the argument contract)."""
import pytest
import torch

from gdn_hip import gdn_decode, gdn_prefill
from gdn_hip.inputs import decode_inputs, prefill_inputs


def _dec():
    return decode_inputs(2, seed=0)


def _pre():
    return prefill_inputs([5, 3], seed=0, with_state=True)


def test_decode_cpu_tensors_rejected():
    with pytest.raises(ValueError, match="no CPU path"):
        gdn_decode(*_dec().args())


def test_prefill_cpu_tensors_rejected():
    with pytest.raises(ValueError, match="no CPU path"):
        gdn_prefill(*_pre().args())


@pytest.mark.parametrize("field,bad,exc", [
    ("q", lambda t: t.float(), TypeError),
    ("k", lambda t: t[..., :64], ValueError),
    ("v", lambda t: t[:, :, :24], ValueError),      # 24 v-heads vs 16 q/k heads: not a multiple
    ("state", lambda t: t.double(), TypeError),
    ("A_log", lambda t: t[:3], ValueError),
    ("a", lambda t: t.float(), TypeError),
    ("b", lambda t: t[:, :, :5], ValueError),
    ("dt_bias", lambda t: t.half(), TypeError),
])
def test_decode_bad_arguments(field, bad, exc):
    inp = _dec()
    setattr(inp, field, bad(getattr(inp, field)))
    with pytest.raises(exc):
        gdn_decode(*inp.args())


def test_decode_empty_sequence_rejected():
    inp = decode_inputs(2, seed=0)
    for f in ("q", "k", "v", "a", "b"):
        setattr(inp, f, getattr(inp, f)[:, :0])
    with pytest.raises(ValueError, match="seq_len"):
        gdn_decode(*inp.args())


def test_decode_head_size_rejected():
    inp = decode_inputs(2, d=64, seed=0)
    with pytest.raises(ValueError, match="head_size"):
        gdn_decode(*inp.args())


@pytest.mark.parametrize("field,bad,exc", [
    ("q", lambda t: t.unsqueeze(0), ValueError),
    ("cu_seqlens", lambda t: t.float(), TypeError),
    ("cu_seqlens", lambda t: t.view(1, -1), ValueError),
    ("state", lambda t: t[:1], ValueError),
    ("a", lambda t: t[:-1], ValueError),
])
def test_prefill_bad_arguments(field, bad, exc):
    inp = _pre()
    setattr(inp, field, bad(getattr(inp, field)))
    with pytest.raises(exc):
        gdn_prefill(*inp.args())


def test_output_buffers_validated():
    inp = _dec()
    with pytest.raises(ValueError):
        gdn_decode(*inp.args(), output=torch.empty(2, 1, 32, 64, dtype=torch.bfloat16))
    inp = _pre()
    with pytest.raises(TypeError):
        gdn_prefill(*inp.args(), new_state=torch.empty(2, 32, 128, 128, dtype=torch.float16))
