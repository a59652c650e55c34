"""MI355X-native routed-expert MoE hot path (router, dispatch, quantized
SwiGLU experts, combine, HBM expert slab and slot table).

Host code calls hand-written gfx950 HIP kernels through the C ABI in
include/pmoe.h (libpmoe.so, built in-tree).
"""

from ._lib import PmoeError, geom, lib  # noqa: F401

__all__ = ["PmoeError", "geom", "lib"]
