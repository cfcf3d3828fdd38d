"""sapphire_amd: MI355X-native (gfx950) quantized decode path of Sapphire.

The product is the C-ABI library ``libsapphire_hip.so`` (headers in ``include/``).
This package builds it, loads it through ctypes and offers thin numpy-facing helpers
for tests and benchmarks. Importing :data:`lib` raises if the library was not built:
there is no CPU fallback.
"""
from __future__ import annotations

import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsapphire_hip.so")

__all__ = ["LIB_PATH", "load"]


def load():
    """Load libsapphire_hip.so (ctypes.CDLL with prototypes); raises if missing."""
    from ._lib import load_library
    return load_library(LIB_PATH)
