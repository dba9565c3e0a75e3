"""gefen: the Gefen optimizer family with an MI355X-native fused step.

Drop-in for the reference package's public surface (src/gefen/__init__.py):
the optimizer classes keep their constructor arguments, param-group layout and
state_dict format; the fused step runs hand-written gfx950 HIP kernels through
the C ABI in include/gefenx.h.
"""
from gefen.gefen import Gefen

__all__ = ["Gefen"]
