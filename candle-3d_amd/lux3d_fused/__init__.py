"""lux3d_fused: MI355X (gfx950) fused transformer-layer ops for candle-3d.

`ops` mirrors candle-3d's Tensor-level operator surface; `_lib` is the
ctypes binding of the C ABI (include/lux3d_fused.h); `synth` generates the
seeded inputs used by the tests and the benchmark.
"""
from . import _lib  # noqa: F401  (fails loudly when liblux3d_fused.so is missing)
from ._lib import ABI_VERSION, LIB_PATH, Lux3dError  # noqa: F401

__all__ = ["ABI_VERSION", "LIB_PATH", "Lux3dError"]
