"""ctypes binding of the C ABI in include/gdn_hip.h.

torch is imported before the library is opened so that libgdn_hip.so binds to
the HIP runtime torch already loaded (both carry the soname libamdhip64.so.7):
one runtime per process, so torch's streams and allocations are valid handles
for the kernels.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede CDLL: see module docstring)

from .build import FAST_NAME, LIB_PATH, fast_lib_path

_c_i32 = ctypes.c_int32
_c_i64 = ctypes.c_int64
_c_f32 = ctypes.c_float
_c_ptr = ctypes.c_void_p

ABI_VERSION = 1

GDN_OK = 0
GDN_EINVAL = -1
GDN_ELAYOUT = -2
GDN_EWORKSPACE = -3
GDN_ELAUNCH = -4


class DecodeParams(ctypes.Structure):
    """Mirror of gdn_decode_params."""

    _fields_ = [
        ("struct_size", _c_i32),
        ("batch", _c_i32),
        ("seq_len", _c_i32),
        ("num_qk_heads", _c_i32),
        ("num_v_heads", _c_i32),
        ("head_size", _c_i32),
        ("scale", _c_f32),
        ("variant", _c_i32),
        ("q", _c_ptr), ("q_stride", _c_i64 * 4),
        ("k", _c_ptr), ("k_stride", _c_i64 * 4),
        ("v", _c_ptr), ("v_stride", _c_i64 * 4),
        ("state", _c_ptr), ("state_stride", _c_i64 * 4),
        ("A_log", _c_ptr), ("A_log_stride", _c_i64),
        ("a", _c_ptr), ("a_stride", _c_i64 * 3),
        ("dt_bias", _c_ptr), ("dt_bias_stride", _c_i64),
        ("b", _c_ptr), ("b_stride", _c_i64 * 3),
        ("output", _c_ptr), ("output_stride", _c_i64 * 4),
        ("new_state", _c_ptr), ("new_state_stride", _c_i64 * 4),
    ]


class PrefillParams(ctypes.Structure):
    """Mirror of gdn_prefill_params."""

    _fields_ = [
        ("struct_size", _c_i32),
        ("total_tokens", _c_i32),
        ("num_seqs", _c_i32),
        ("num_qk_heads", _c_i32),
        ("num_v_heads", _c_i32),
        ("head_size", _c_i32),
        ("scale", _c_f32),
        ("cu_seqlens_int64", _c_i32),
        ("variant", _c_i32),
        ("reserved", _c_i32),
        ("q", _c_ptr), ("q_stride", _c_i64 * 3),
        ("k", _c_ptr), ("k_stride", _c_i64 * 3),
        ("v", _c_ptr), ("v_stride", _c_i64 * 3),
        ("state", _c_ptr), ("state_stride", _c_i64 * 4),
        ("A_log", _c_ptr), ("A_log_stride", _c_i64),
        ("a", _c_ptr), ("a_stride", _c_i64 * 2),
        ("dt_bias", _c_ptr), ("dt_bias_stride", _c_i64),
        ("b", _c_ptr), ("b_stride", _c_i64 * 2),
        ("cu_seqlens", _c_ptr),
        ("output", _c_ptr), ("output_stride", _c_i64 * 3),
        ("new_state", _c_ptr), ("new_state_stride", _c_i64 * 4),
        ("workspace", _c_ptr),
        ("workspace_bytes", _c_i64),
    ]


# Symbols include/gdn_hip.h declares (tests check the library exports each one).
EXPORTED = (
    "gdn_abi_version",
    "gdn_last_error",
    "gdn_decode_launch",
    "gdn_prefill_workspace_size",
    "gdn_prefill_launch",
    "gdn_prefill_noalloc_capacity",
    "gdn_prefill_launch_noalloc",
)

_lib = None
_lock = threading.Lock()


def load() -> ctypes.CDLL:
    """Open libgdn_hip.so (built by gdn_hip.build / __graft_entry__.build()).

    Raises RuntimeError when the library is missing: there is no fallback path."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run __graft_entry__.build() "
                "(hipcc --offload-arch=gfx950). There is no non-HIP fallback.")
        lib = ctypes.CDLL(LIB_PATH)
        lib.gdn_abi_version.restype = ctypes.c_int
        lib.gdn_abi_version.argtypes = []
        lib.gdn_last_error.restype = ctypes.c_char_p
        lib.gdn_last_error.argtypes = []
        lib.gdn_decode_launch.restype = ctypes.c_int
        lib.gdn_decode_launch.argtypes = [ctypes.POINTER(DecodeParams), _c_ptr]
        lib.gdn_prefill_workspace_size.restype = _c_i64
        lib.gdn_prefill_workspace_size.argtypes = [_c_i32] * 5
        lib.gdn_prefill_launch.restype = ctypes.c_int
        lib.gdn_prefill_launch.argtypes = [ctypes.POINTER(PrefillParams), _c_ptr]
        lib.gdn_prefill_noalloc_capacity.restype = _c_i64
        lib.gdn_prefill_noalloc_capacity.argtypes = []
        lib.gdn_prefill_launch_noalloc.restype = ctypes.c_int
        lib.gdn_prefill_launch_noalloc.argtypes = [ctypes.POINTER(PrefillParams), _c_ptr]
        ver = lib.gdn_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"libgdn_hip.so ABI {ver} != binding ABI {ABI_VERSION}")
        _lib = lib
        return lib


_fast = None
_fast_tried = False


def fast():
    """The per-call fast path module (csrc/gdn_fast_path.cpp), initialised with this
    library's entry points; None when it is not built (the Python path then validates
    and marshals every call itself)."""
    global _fast, _fast_tried
    if _fast_tried:
        return _fast
    lib = load()  # takes _lock itself: before, not inside, the block below
    with _lock:
        if not _fast_tried:
            path = fast_lib_path()
            if path is not None:
                import importlib.machinery
                import importlib.util

                loader = importlib.machinery.ExtensionFileLoader(FAST_NAME, path)
                spec = importlib.util.spec_from_loader(FAST_NAME, loader)
                mod = importlib.util.module_from_spec(spec)
                loader.exec_module(mod)
                addr = lambda f: ctypes.cast(f, ctypes.c_void_p).value  # noqa: E731
                mod.init(addr(lib.gdn_decode_launch), addr(lib.gdn_prefill_launch),
                         addr(lib.gdn_prefill_workspace_size), addr(lib.gdn_last_error))
                _fast = mod
            _fast_tried = True
    return _fast


def last_error() -> str:
    return load().gdn_last_error().decode(errors="replace")


def check(rc: int, what: str) -> None:
    if rc != GDN_OK:
        raise RuntimeError(f"{what} failed (code {rc}): {last_error()}")
