"""Drop-in host entry points with the reference's signatures.

* ``gdn_decode``  <- gdn_decode/solution/triton/kernel.py:221-272
* ``gdn_prefill`` <- gdn_prefill/solution/triton/kernel.py:253-337

Both follow the reference's destination-passing contract: inputs positionally in
definition order, then optional preallocated ``output`` / ``new_state``; both
return ``(output, new_state)``. The arithmetic runs only in the HIP kernels of
libgdn_hip.so, launched on torch's current stream of the inputs' device. There
is no CPU or framework fallback: a missing library or a non-GPU tensor raises.
"""
from __future__ import annotations

import ctypes
import math
import threading

import torch

from . import _lib

_D = 128


# ----------------------------------------------------------------------------- validation helpers
def _need_tensor(name, t, dtype, ndim):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if t.dim() != ndim:
        raise ValueError(f"{name} must have {ndim} dims, got shape {tuple(t.shape)}")


def _need_shape(name, t, shape):
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")


def _need_device(dev, **tensors):
    if dev.type != "cuda":
        raise ValueError("GDN kernels need tensors on a HIP device (torch 'cuda'); "
                         f"got {dev}. There is no CPU path.")
    for name, t in tensors.items():
        if t is not None and t.device != dev:
            raise ValueError(f"{name} is on {t.device}, expected {dev}")


def _resolve_scale(scale, D):
    # gdn_decode/solution/triton/kernel.py:241-242; gdn_prefill/solution/triton/kernel.py:276-277
    if scale is None:
        return 1.0 / math.sqrt(D)
    if isinstance(scale, torch.Tensor):
        # the reference types scale as a float (gdn_decode/solution/triton/kernel.py:230);
        # a device tensor is read back, a host sync a captured graph cannot record
        if scale.is_cuda and torch.cuda.is_current_stream_capturing():
            raise ValueError("scale must be a Python float while a HIP graph is being "
                             "captured (a tensor scale is read back with a device sync)")
        scale = float(scale.item())
    scale = float(scale)
    return 1.0 / math.sqrt(D) if scale == 0.0 else scale


def _layout_ok(t, align_bytes, stride_mult):
    if t.stride(-1) != 1 and t.shape[-1] != 1:
        return False
    if t.data_ptr() % align_bytes:
        return False
    return all(s % stride_mult == 0 for s, n in zip(t.stride()[:-1], t.shape[:-1]) if n > 1)


def _in(t, align_bytes=1, stride_mult=1):
    """Input as the kernels accept it (unit inner stride, alignment): no copy when it
    already is, else a contiguous device copy."""
    if t is None or _layout_ok(t, align_bytes, stride_mult):
        return t
    return t.contiguous()


def _strides(t, n):
    if t is None:
        return (0,) * n
    st = list(t.stride())
    # a size-1 innermost dim may report any stride; the ABI wants 1
    if t.shape[-1] == 1:
        st[-1] = 1
    return tuple(st)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(dev):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


# ----------------------------------------------------------------------------- decode
def _decode_marshal(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state):
    """Validate like the reference host wrapper and build the ABI params.

    Returns (params, output, new_state, copy_back, keep): copy_back lists
    (user_tensor, kernel_tensor) pairs to copy after the launch (only when a user
    buffer's layout is not one the kernel writes directly); keep holds every tensor
    the params point at, so they outlive the launch."""
    _need_tensor("q", q, torch.bfloat16, 4)
    B, T, HQK, D = q.shape
    _need_tensor("k", k, torch.bfloat16, 4)
    _need_shape("k", k, (B, T, HQK, D))
    _need_tensor("v", v, torch.bfloat16, 4)
    HV = v.shape[2]
    _need_shape("v", v, (B, T, HV, D))
    if D != _D:
        raise ValueError(f"head_size {D} unsupported: the kernels are built for D={_D}")
    if HV % HQK != 0:
        raise ValueError(f"num_v_heads ({HV}) must be a multiple of num_q_heads ({HQK})")
    if T < 1:
        raise ValueError(f"seq_len must be >= 1 (got {T})")
    if state is not None:
        _need_tensor("state", state, torch.float32, 4)
        _need_shape("state", state, (B, HV, D, D))
    _need_tensor("A_log", A_log, torch.float32, 1)
    _need_shape("A_log", A_log, (HV,))
    _need_tensor("a", a, torch.bfloat16, 3)
    _need_shape("a", a, (B, T, HV))
    _need_tensor("dt_bias", dt_bias, torch.float32, 1)
    _need_shape("dt_bias", dt_bias, (HV,))
    _need_tensor("b", b, torch.bfloat16, 3)
    _need_shape("b", b, (B, T, HV))
    if output is not None:
        _need_tensor("output", output, torch.bfloat16, 4)
        _need_shape("output", output, (B, T, HV, D))
    if new_state is not None:
        _need_tensor("new_state", new_state, torch.float32, 4)
        _need_shape("new_state", new_state, (B, HV, D, D))
    dev = q.device
    _need_device(dev, k=k, v=v, state=state, A_log=A_log, a=a, dt_bias=dt_bias, b=b,
                 output=output, new_state=new_state)
    scale = _resolve_scale(scale, D)

    # gdn_decode/solution/triton/kernel.py:243-247 (state=None needs no zero buffer:
    # the kernel skips the read)
    if output is None:
        output = torch.empty((B, T, HV, D), dtype=torch.bfloat16, device=dev)
    if new_state is None:
        new_state = torch.empty((B, HV, D, D), dtype=torch.float32, device=dev)

    qk_ok = (8, 4)
    st_ok = (16, 4)
    q_, k_ = _in(q, *qk_ok), _in(k, *qk_ok)
    v_, a_, b_ = _in(v), _in(a), _in(b)
    st_ = _in(state, *st_ok)
    copy_back = []
    out_ = output
    if not _layout_ok(output, 2, 1):
        out_ = torch.empty((B, T, HV, D), dtype=torch.bfloat16, device=dev)
        copy_back.append((output, out_))
    ns_ = new_state
    if not _layout_ok(new_state, *st_ok):
        ns_ = torch.empty((B, HV, D, D), dtype=torch.float32, device=dev)
        copy_back.append((new_state, ns_))
    # in place needs identical strides, and seq_len 1: with T > 1 every token reads the
    # input state while the last one writes new_state
    if st_ is not None and st_.data_ptr() == ns_.data_ptr() and (
            T > 1 or st_.stride() != ns_.stride()):
        st_ = st_.clone()

    P = _lib.DecodeParams()
    P.struct_size = ctypes.sizeof(_lib.DecodeParams)
    P.batch, P.seq_len, P.num_qk_heads, P.num_v_heads, P.head_size = B, T, HQK, HV, D
    P.scale = scale
    P.variant = 0
    P.q, P.q_stride = _ptr(q_), _strides(q_, 4)
    P.k, P.k_stride = _ptr(k_), _strides(k_, 4)
    P.v, P.v_stride = _ptr(v_), _strides(v_, 4)
    P.state, P.state_stride = _ptr(st_), _strides(st_, 4)
    P.A_log, P.A_log_stride = _ptr(A_log), A_log.stride(0)
    P.a, P.a_stride = _ptr(a_), _strides(a_, 3)
    P.dt_bias, P.dt_bias_stride = _ptr(dt_bias), dt_bias.stride(0)
    P.b, P.b_stride = _ptr(b_), _strides(b_, 3)
    P.output, P.output_stride = _ptr(out_), _strides(out_, 4)
    P.new_state, P.new_state_stride = _ptr(ns_), _strides(ns_, 4)
    # keep every tensor the params point at alive as long as the params
    keep = (q_, k_, v_, st_, A_log, a_, dt_bias, b_, out_, ns_)
    return P, output, new_state, copy_back, keep


def gdn_decode(q, k, v, state, A_log, a, dt_bias, b, scale, output=None, new_state=None):
    """Gated DeltaNet decode (k-last fp32 state).

    q, k: bf16 [B, T, HQK, D]; v: bf16 [B, T, HV, D]; state: fp32 [B, HV, D, D] or None
    (zeros); A_log, dt_bias: fp32 [HV]; a, b: bf16 [B, T, HV]; scale: float (None/0 ->
    1/sqrt(D)). Returns (output bf16 [B, T, HV, D], new_state fp32 [B, HV, D, D]);
    ``new_state`` may be ``state`` itself (in-place update).
    T is 1 in the reference's workloads. For T > 1 each token is one step from the input
    state, as the reference kernel's per-token programs compute it
    (gdn_decode/solution/triton/kernel.py:117-118,146-147); new_state is the last token's
    update (the reference lets every token store it, in no fixed order).
    Mirrors gdn_decode/solution/triton/kernel.py:221-272 (defaults at :238-247).
    Destination-passing calls (output and new_state given) whose buffers the kernel can
    use in place are validated and launched by the C++ fast path; every other call goes
    through the Python validation below, which raises the wrapper's errors.
    """
    if output is not None and new_state is not None and (scale is None or type(scale) is float):
        fast = _lib.fast()
        if fast is not None and fast.decode(q, k, v, state, A_log, a, dt_bias, b,
                                            0.0 if scale is None else scale, output,
                                            new_state, 0) == 0:
            return output, new_state
    with torch.no_grad():
        P, output, new_state, copy_back, _keep = _decode_marshal(
            q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state)
        if P.batch == 0:
            return output, new_state
        dev = q.device
        lib = _lib.load()
        with torch.cuda.device(dev):
            _lib.check(lib.gdn_decode_launch(ctypes.byref(P), _stream(dev)), "gdn_decode_launch")
        for user, tmp in copy_back:
            user.copy_(tmp)
    return output, new_state


class DecodePlan:
    """A validated, pre-marshalled decode launch over fixed tensors.

    For loops that call the same shapes and buffers every step (serving, the
    benchmark): the reference-style validation runs once here and ``run()`` is a
    single ABI call on the current stream. The buffers must already have layouts
    the kernel reads and writes directly (no staging copies)."""

    def __init__(self, q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state):
        P, out, ns, copy_back, keep = _decode_marshal(q, k, v, state, A_log, a, dt_bias, b,
                                                      scale, output, new_state)
        if copy_back or any(x is not y for x, y in zip(keep[:8], (q, k, v, state, A_log, a,
                                                                  dt_bias, b))):
            raise ValueError("DecodePlan needs buffers the kernel can use in place")
        self._P, self._keep, self.output, self.new_state = P, keep, out, ns
        self._pref = ctypes.byref(P)
        self._dev_index = q.device.index
        self._launch = _lib.load().gdn_decode_launch

    def run(self):
        stream = torch._C._cuda_getCurrentRawStream(self._dev_index)
        _lib.check(self._launch(self._pref, stream), "gdn_decode_launch")
        return self.output, self.new_state


# ----------------------------------------------------------------------------- prefill
_prefill_variant = 0


def set_prefill_variant(v: int) -> None:
    """Select a prefill kernel variant: 0 = tuned default; 1 / 2 scan every sequence whole
    with 4 / 8 scan waves per workgroup (no segments)."""
    global _prefill_variant
    _prefill_variant = int(v)


_ws_lock = threading.Lock()
_ws_cache: dict = {}
_graph_ws: list = []


def _workspace(dev, stream, nbytes):
    """Device workspace for one prefill call.

    Eager calls share a grow-only buffer per (device, stream), rewritten by every call
    (stream order keeps calls on one stream apart). A call being captured into a HIP
    graph gets a buffer of its own, kept until ``release_workspace(graphs=True)``: the
    graph's kernels keep pointing at it for as long as the graph may be replayed, and
    graphs captured on the shared capture stream must not share (or free) one another's
    workspace. Each capture adds one (about 72 MB at 8K tokens in 16 sequences), so a
    caller that captures many graphs releases them once it has destroyed those graphs,
    or uses gdn_prefill_launch_noalloc, whose workspace is one static array."""
    if torch.cuda.is_current_stream_capturing():
        buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=dev)
        with _ws_lock:
            _graph_ws.append(buf)
        return buf
    key = (dev.index, stream.cuda_stream)
    with _ws_lock:
        buf = _ws_cache.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
            _ws_cache[key] = buf
        return buf


def graph_workspace_bytes() -> int:
    """Bytes held by the workspaces of captured prefills (see ``release_workspace``)."""
    with _ws_lock:
        return sum(b.numel() for b in _graph_ws)


def release_workspace(graphs: bool = False) -> None:
    """Drop the cached eager prefill workspaces, the Python path's and the fast path's
    (they return to torch's caching allocator; the caller synchronises first, so that no
    call in flight still uses them). With ``graphs=True`` also drop the workspaces of every
    prefill captured into a HIP graph so far: only once every graph that holds such a
    prefill has been destroyed (replaying one afterwards reads freed memory)."""
    with _ws_lock:
        _ws_cache.clear()
        if graphs:
            _graph_ws.clear()
    fast = _lib.fast()
    if fast is not None:
        fast.release_workspace()


def _prefill_marshal(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output,
                     new_state, with_workspace=True):
    """Validate like the reference host wrapper and build the ABI params.

    Returns ((output, new_state),) when there is nothing to launch (empty input, handled
    here as gdn_prefill/solution/triton/kernel.py:286-302 does), else (params, output,
    new_state, copy_back, keep, stream) as _decode_marshal does. ``with_workspace=False``
    leaves the workspace fields empty (for gdn_prefill_launch_noalloc)."""
    _need_tensor("q", q, torch.bfloat16, 3)
    T, HQK, D = q.shape
    _need_tensor("k", k, torch.bfloat16, 3)
    _need_shape("k", k, (T, HQK, D))
    _need_tensor("v", v, torch.bfloat16, 3)
    HV = v.shape[1]
    _need_shape("v", v, (T, HV, D))
    if D != _D:
        raise ValueError(f"head_size {D} unsupported: the kernels are built for D={_D}")
    if HV % HQK != 0:
        raise ValueError(f"num_v_heads ({HV}) must be a multiple of num_q_heads ({HQK})")
    if not isinstance(cu_seqlens, torch.Tensor) or cu_seqlens.dtype not in (torch.int32,
                                                                           torch.int64):
        raise TypeError("cu_seqlens must be an int32 or int64 tensor")
    if cu_seqlens.dim() != 1 or cu_seqlens.shape[0] < 1:
        raise ValueError("cu_seqlens must be 1-D with N+1 >= 1 entries")
    N = cu_seqlens.shape[0] - 1
    if state is not None:
        _need_tensor("state", state, torch.float32, 4)
        _need_shape("state", state, (N, HV, D, D))
    _need_tensor("A_log", A_log, torch.float32, 1)
    _need_shape("A_log", A_log, (HV,))
    _need_tensor("a", a, torch.bfloat16, 2)
    _need_shape("a", a, (T, HV))
    _need_tensor("dt_bias", dt_bias, torch.float32, 1)
    _need_shape("dt_bias", dt_bias, (HV,))
    _need_tensor("b", b, torch.bfloat16, 2)
    _need_shape("b", b, (T, HV))
    HO = max(HQK, HV)  # output heads: gdn_prefill/solution/triton/kernel.py:267,283
    if output is not None:
        _need_tensor("output", output, torch.bfloat16, 3)
        _need_shape("output", output, (T, HO, D))
    if new_state is not None:
        _need_tensor("new_state", new_state, torch.float32, 4)
        _need_shape("new_state", new_state, (N, HV, D, D))
    dev = q.device
    _need_device(dev, k=k, v=v, state=state, A_log=A_log, a=a, dt_bias=dt_bias, b=b,
                 cu_seqlens=cu_seqlens, output=output, new_state=new_state)
    scale = _resolve_scale(scale, D)

    if output is None:
        output = torch.empty((T, HO, D), dtype=torch.bfloat16, device=dev)
    if new_state is None:
        new_state = torch.empty((N, HV, D, D), dtype=torch.float32, device=dev)
    if N == 0 or T == 0:
        # gdn_prefill/solution/triton/kernel.py:286-302: zeroed output, state copied
        output.zero_()
        if state is None:
            new_state.zero_()
        elif new_state.data_ptr() != state.data_ptr():
            new_state.copy_(state)
        return ((output, new_state),)

    qk_ok = (16, 8)
    st_ok = (16, 4)
    q_, k_, v_ = _in(q, *qk_ok), _in(k, *qk_ok), _in(v, *qk_ok)
    a_, b_ = _in(a), _in(b)
    cu_ = cu_seqlens.contiguous()
    st_ = _in(state, *st_ok)
    out_ = output if _layout_ok(output, 16, 8) else torch.empty(
        (T, HO, D), dtype=torch.bfloat16, device=dev)
    ns_ = new_state if _layout_ok(new_state, *st_ok) else torch.empty(
        (N, HV, D, D), dtype=torch.float32, device=dev)
    if st_ is not None and st_.data_ptr() == ns_.data_ptr() and st_.stride() != ns_.stride():
        st_ = st_.clone()

    lib = _lib.load()
    stream = torch.cuda.current_stream(dev)
    ws = None
    if with_workspace:
        ws_bytes = int(lib.gdn_prefill_workspace_size(T, N, HQK, HV, D))
        if ws_bytes < 0:
            raise RuntimeError(f"gdn_prefill_workspace_size failed: {_lib.last_error()}")
        ws = _workspace(dev, stream, ws_bytes)

    P = _lib.PrefillParams()
    P.struct_size = ctypes.sizeof(_lib.PrefillParams)
    P.total_tokens, P.num_seqs, P.num_qk_heads, P.num_v_heads, P.head_size = T, N, HQK, HV, D
    P.scale = scale
    P.cu_seqlens_int64 = 1 if cu_.dtype == torch.int64 else 0
    P.variant = _prefill_variant
    P.q, P.q_stride = _ptr(q_), _strides(q_, 3)
    P.k, P.k_stride = _ptr(k_), _strides(k_, 3)
    P.v, P.v_stride = _ptr(v_), _strides(v_, 3)
    P.state, P.state_stride = _ptr(st_), _strides(st_, 4)
    P.A_log, P.A_log_stride = _ptr(A_log), A_log.stride(0)
    P.a, P.a_stride = _ptr(a_), _strides(a_, 2)
    P.dt_bias, P.dt_bias_stride = _ptr(dt_bias), dt_bias.stride(0)
    P.b, P.b_stride = _ptr(b_), _strides(b_, 2)
    P.cu_seqlens = _ptr(cu_)
    P.output, P.output_stride = _ptr(out_), _strides(out_, 3)
    P.new_state, P.new_state_stride = _ptr(ns_), _strides(ns_, 4)
    P.workspace, P.workspace_bytes = (_ptr(ws), ws.numel()) if ws is not None else (None, 0)
    copy_back = [(u, t) for u, t in ((output, out_), (new_state, ns_)) if t is not u]
    keep = (q_, k_, v_, st_, A_log, a_, dt_bias, b_, cu_, out_, ns_, ws)
    return P, output, new_state, copy_back, keep, stream


def gdn_prefill(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output=None,
                new_state=None):
    """Gated DeltaNet prefill over packed variable-length sequences.

    q, k: bf16 [T, HQK, D]; v: bf16 [T, HV, D]; state: fp32 [N, HV, D, D] or None;
    A_log, dt_bias: fp32 [HV]; a, b: bf16 [T, HV]; cu_seqlens: int32/int64 [N+1];
    scale: float (None/0 -> 1/sqrt(D)). Returns (output bf16 [T, max(HQK,HV), D],
    new_state fp32 [N, HV, D, D]).
    Mirrors gdn_prefill/solution/triton/kernel.py:253-337 (argument order :254,
    defaults and DPS handling :276-302), generalised from the 4/8 head layout it
    asserts (:271-274) to any HV that is a multiple of HQK.
    Destination-passing calls outside graph capture whose buffers the kernels can use in
    place are validated and launched by the C++ fast path (with its own per-stream
    workspace cache); every other call goes through the Python validation below.
    """
    if output is not None and new_state is not None and (scale is None or type(scale) is float):
        fast = _lib.fast()
        if fast is not None and fast.prefill(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens,
                                             0.0 if scale is None else scale, output,
                                             new_state, _prefill_variant) == 0:
            return output, new_state
    with torch.no_grad():
        m = _prefill_marshal(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output,
                             new_state)
        if len(m) == 1:  # nothing to launch
            return m[0]
        P, output, new_state, copy_back, _keep, stream = m
        with torch.cuda.device(q.device):
            _lib.check(_lib.load().gdn_prefill_launch(ctypes.byref(P),
                                                      ctypes.c_void_p(stream.cuda_stream)),
                       "gdn_prefill_launch")
        for user, tmp in copy_back:
            user.copy_(tmp)
    return output, new_state
