"""CPU tests of the C ABI: the library loads, exports every symbol include/gdn_hip.h
declares, agrees with the ctypes struct layout, and rejects bad arguments with an
error code and message before touching any device memory."""
import ctypes
import os
import re
import subprocess
import tempfile

import pytest

from gdn_hip import _lib
from gdn_hip.build import INCLUDE, LIB_PATH

HEADER = os.path.join(INCLUDE, "gdn_hip.h")


def _declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(gdn_[a-z0-9_]+)\s*\(", src)))


def test_library_built():
    assert os.path.exists(LIB_PATH), "run __graft_entry__.build() first"


def test_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB_PATH)
    declared = _declared_functions()
    assert set(declared) == set(_lib.EXPORTED), declared
    for name in declared:
        assert hasattr(lib, name), f"{name} not exported"
    nm = subprocess.run(["nm", "-D", "--defined-only", LIB_PATH], capture_output=True,
                        text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in nm.splitlines() if " T " in ln}
    assert set(declared) <= exported


def test_abi_version():
    assert _lib.load().gdn_abi_version() == _lib.ABI_VERSION


def test_struct_layout_matches_header():
    """Compile a probe against the header and compare sizeof/offsetof with ctypes."""
    fields = {
        "gdn_decode_params": _lib.DecodeParams,
        "gdn_prefill_params": _lib.PrefillParams,
    }
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "gdn_hip.h"',
             "int main(void) {"]
    for cname, cls in fields.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0; }")
    with tempfile.TemporaryDirectory() as td:
        c = os.path.join(td, "probe.c")
        exe = os.path.join(td, "probe")
        open(c, "w").write("\n".join(lines))
        subprocess.run(["gcc", "-std=c11", f"-I{INCLUDE}", c, "-o", exe], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout
    got = {}
    for ln in out.splitlines():
        cname, fname, val = ln.split()
        got[(cname, fname)] = int(val)
    for cname, cls in fields.items():
        assert got[(cname, "size")] == ctypes.sizeof(cls), cname
        for fname, _ in cls._fields_:
            assert got[(cname, fname)] == getattr(cls, fname).offset, (cname, fname)


def test_decode_rejects_bad_params_without_launch():
    lib = _lib.load()
    P = _lib.DecodeParams()
    P.struct_size = 3  # wrong size
    rc = lib.gdn_decode_launch(ctypes.byref(P), None)
    assert rc == _lib.GDN_EINVAL
    assert "struct_size" in _lib.last_error()
    P.struct_size = ctypes.sizeof(_lib.DecodeParams)
    P.batch, P.seq_len, P.num_qk_heads, P.num_v_heads, P.head_size = 2, 1, 16, 32, 64
    assert lib.gdn_decode_launch(ctypes.byref(P), None) == _lib.GDN_EINVAL
    assert "head_size" in _lib.last_error()
    P.head_size, P.seq_len = 128, 0
    assert lib.gdn_decode_launch(ctypes.byref(P), None) == _lib.GDN_EINVAL
    assert "seq_len" in _lib.last_error()
    P.seq_len, P.num_v_heads = 1, 24  # 24 % 16 != 0
    assert lib.gdn_decode_launch(ctypes.byref(P), None) == _lib.GDN_EINVAL
    P.num_qk_heads, P.num_v_heads = 1, 65536  # v-heads are a grid dimension (<= 65535)
    assert lib.gdn_decode_launch(ctypes.byref(P), None) == _lib.GDN_EINVAL
    assert "65535" in _lib.last_error()
    P.num_qk_heads, P.num_v_heads = 16, 32  # valid sizes but NULL tensors
    assert lib.gdn_decode_launch(ctypes.byref(P), None) == _lib.GDN_EINVAL
    assert "NULL" in _lib.last_error()
    P.batch = 0  # empty batch is a no-op success
    assert lib.gdn_decode_launch(ctypes.byref(P), None) == _lib.GDN_OK
    P.variant = 3  # only the tuned kernel is built
    assert lib.gdn_decode_launch(ctypes.byref(P), None) == _lib.GDN_EINVAL
    assert "variant" in _lib.last_error()


def test_prefill_rejects_unknown_variant_without_launch():
    lib = _lib.load()
    P = _lib.PrefillParams()
    P.struct_size = ctypes.sizeof(_lib.PrefillParams)
    P.total_tokens, P.num_seqs, P.num_qk_heads, P.num_v_heads, P.head_size = 64, 1, 16, 32, 128
    P.variant = 3
    assert lib.gdn_prefill_launch(ctypes.byref(P), None) == _lib.GDN_EINVAL
    assert "variant" in _lib.last_error()


def test_decode_rejects_bad_layout_without_launch():
    """Layout checks run before any launch: fake (never dereferenced) pointers suffice."""
    lib = _lib.load()
    P = _lib.DecodeParams()
    P.struct_size = ctypes.sizeof(_lib.DecodeParams)
    P.batch, P.seq_len, P.num_qk_heads, P.num_v_heads, P.head_size = 2, 1, 16, 32, 128
    fake = 0x10000
    for f in ("q", "k", "v", "A_log", "a", "dt_bias", "b", "output", "new_state"):
        setattr(P, f, fake)
    P.q_stride = (2048, 2048, 128, 2)  # innermost stride 2
    rc = lib.gdn_decode_launch(ctypes.byref(P), None)
    assert rc == _lib.GDN_ELAYOUT and "innermost" in _lib.last_error()
    P.q_stride = (2048, 2048, 128, 1)
    P.k_stride = (2048, 2048, 128, 1)
    P.v_stride = P.output_stride = (4096, 4096, 128, 1)
    P.new_state_stride = (32 * 16384, 16384, 128, 1)
    P.new_state = fake + 4  # misaligned
    rc = lib.gdn_decode_launch(ctypes.byref(P), None)
    assert rc == _lib.GDN_ELAYOUT and "aligned" in _lib.last_error()
    # seq_len > 1 reads the input state for every token: in place would race
    P.new_state = P.state = fake
    P.state_stride = P.new_state_stride
    P.seq_len = 2
    rc = lib.gdn_decode_launch(ctypes.byref(P), None)
    assert rc == _lib.GDN_EINVAL and "alias" in _lib.last_error()


def test_prefill_workspace_size_rejects_bad_sizes():
    lib = _lib.load()
    assert lib.gdn_prefill_workspace_size(-1, 1, 16, 32, 128) < 0
    assert lib.gdn_prefill_workspace_size(100, 1, 16, 24, 128) < 0
    assert lib.gdn_prefill_workspace_size(100, 1, 16, 32, 64) < 0
    assert lib.gdn_prefill_workspace_size(4096, 1, 16, 32, 128) > 0


def test_one_hip_runtime_in_process():
    """torch and libgdn_hip.so share one libamdhip64 (same soname, loaded once)."""
    _lib.load()
    maps = open("/proc/self/maps").read()
    libs = {ln.split()[-1] for ln in maps.splitlines() if "libamdhip64" in ln}
    assert len(libs) == 1, libs


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    """No fallback: an absent library raises instead of computing anything."""
    import gdn_hip._lib as L

    monkeypatch.setattr(L, "_lib", None)
    monkeypatch.setattr(L, "LIB_PATH", str(tmp_path / "absent.so"))
    with pytest.raises(RuntimeError, match="not built"):
        L.load()


def test_fast_path_extension_loads_and_declines_host_tensors():
    """The C++ per-call fast path loads next to the library (from any thread, without
    deadlocking on the loader's lock) and declines tensors that are not on a HIP device,
    which the Python path then rejects."""
    import threading

    import torch

    from gdn_hip import _lib

    res = []
    th = threading.Thread(target=lambda: res.append(_lib.fast()))
    th.start()
    th.join(timeout=60)
    assert not th.is_alive(), "loading the fast path hung"
    fast = res[0]
    assert fast is not None, "fast-path extension not built (gdn_hip.build.build_fast)"
    assert _lib.fast() is fast
    t = lambda *s: torch.zeros(s, dtype=torch.bfloat16)  # noqa: E731
    f = lambda *s: torch.zeros(s, dtype=torch.float32)  # noqa: E731
    assert fast.decode(t(1, 1, 4, 128), t(1, 1, 4, 128), t(1, 1, 8, 128), f(1, 8, 128, 128),
                       f(8), t(1, 1, 8), f(8), t(1, 1, 8), 0.5, t(1, 1, 8, 128),
                       f(1, 8, 128, 128), 0) == 1


def test_native_caller_loads_and_links():
    """The native C++ caller (tests/native) resolves the library, the oracle and the HIP
    runtime through its run paths; without a GPU it stops at the device check (77)."""
    exe = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native", "gdn_native_caller")
    assert os.path.exists(exe), "run __graft_entry__.build()"
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode in (0, 77), r.stdout + r.stderr
    if r.returncode == 77:
        assert "no HIP device" in r.stdout
