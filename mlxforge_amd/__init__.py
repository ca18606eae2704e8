"""mlxforge_amd -- MI355X-native batched token sampler (drop-in for mlxforge's src/sample).

The product is libmlxf_sampler.so (C ABI: include/mlxf_sampler.h), hand-written
HIP for gfx950.  This package holds its sources (csrc/), the build recipe
(build.py), the C++ host wrapper (include/mlxforge_amd/sampler.hpp) and a
Python mirror of the sampler interface (sampler.py) over the same C ABI.
"""
from . import _lib  # noqa: F401

__all__ = ["sampler", "workloads"]
