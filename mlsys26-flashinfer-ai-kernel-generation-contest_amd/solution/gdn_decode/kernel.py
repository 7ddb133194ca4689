"""Entry module a flashinfer-bench style harness imports (``kernel.py::<entry>``).

It re-exports the HIP-backed entry points with the reference signatures and builds
libgdn_hip.so (hipcc, gfx950) on first import when it is not built yet.
"""
import os
import sys

_HERE = os.path.dirname(os.path.abspath(__file__))
# packed layout: kernel.py next to gdn_hip/; in-repo layout: solution/<name>/kernel.py
for _root in (_HERE, os.path.dirname(os.path.dirname(_HERE))):
    if os.path.isdir(os.path.join(_root, "gdn_hip")):
        if _root not in sys.path:
            sys.path.insert(0, _root)
        break

from gdn_hip import build as _build  # noqa: E402

if not os.path.exists(_build.LIB_PATH):
    _build.build()

from gdn_hip import gdn_decode, gdn_prefill  # noqa: E402,F401
