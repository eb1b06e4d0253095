"""lightning_core -- Python surface of the MI355X (gfx950) backend.

Mirrors the reference's pybind module for the dense forward path
(python/bindings/bind_attention.cpp, bind_ops.cpp, bind_runtime.cpp,
bind_integrated.cpp): same function names, argument names and error behaviour
(`RuntimeError` carrying the status string for a non-success status,
`ValueError` for shape errors).  Differences, all deliberate:

* the default device is "hip" (the only device this library computes on);
  "cpu", "cuda" and "metal" are accepted and answer "not supported";
* half-precision compute is an explicit `compute_dtype` argument on the new
  batched-attention, resident-matmul and ViT-block entry points.

Everything calls the C ABI in include/lightning_core_hip.h through ctypes;
there is no Python or CPU implementation of any kernel here.
"""
from ._core import *  # noqa: F401,F403
from ._core import __all__ as _core_all
from ._graph import *  # noqa: F401,F403
from ._graph import __all__ as _graph_all
from . import api  # noqa: F401

__all__ = list(_core_all) + list(_graph_all)
