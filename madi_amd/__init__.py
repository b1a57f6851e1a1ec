"""madi_amd -- MI355X (gfx950) Q8 matmul path of the Whisper large-v3-turbo engine.

The product is libmadi_q8.so (HIP kernels behind the C ABI in include/madi_q8.h);
this package holds its sources (csrc/), its build recipe (build.py), a ctypes
binding (_lib.py) and a Python mirror of the engine's operator wrappers (q8.py).
"""
from ._lib import LIB_PATH, MadiError, lib  # noqa: F401

__all__ = ["LIB_PATH", "MadiError", "lib"]
