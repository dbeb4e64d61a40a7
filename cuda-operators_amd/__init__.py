"""kvq -- INT8 KV-cache decode attention for AMD Instinct MI355X (gfx950).

The operator is libkvq.so (HIP kernels + the C ABI in include/kvq.h); this
package is its host-side binding for callers that hold torch device tensors:
  kvq    ctypes binding of every entry point (reference ABI + extension)
  synth  seeded synthetic caches for the benchmark configurations
Import with importlib.import_module("cuda-operators_amd") (the directory name
is not a Python identifier).
"""
from . import kvq  # noqa: F401

__version__ = "0.1.0"
