"""MI355X-native Gated DeltaNet (GDN) layer for the overhang Qwen3.5/3.6 engine.

The product is the C-ABI library ``libom_hip.so`` (declared in
``include/om_hip.h``) built from ``overhang_amd/csrc``; ``overhang_amd.gdn``
is a thin ctypes front-end to it for Python callers, tests and benchmarks.
"""
from .dims import GdnDims, TINY, CFG1, Q35B  # noqa: F401
