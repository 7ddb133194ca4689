"""MI355X (gfx950) Gated DeltaNet decode / prefill behind a C ABI.

``gdn_decode`` and ``gdn_prefill`` keep the signatures of the reference solutions'
entry points (``kernel.py::gdn_decode``, ``kernel.py::gdn_prefill``) and launch
hand-written HIP kernels from libgdn_hip.so.
"""
from .api import gdn_decode, gdn_prefill, graph_workspace_bytes, release_workspace  # noqa: F401

__all__ = ["gdn_decode", "gdn_prefill", "graph_workspace_bytes", "release_workspace"]
