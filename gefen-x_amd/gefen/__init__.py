"""gefen: the Gefen optimizer family with an MI355X-native fused step.

Drop-in for the reference package's public surface (src/gefen/__init__.py):
the optimizer classes keep their constructor arguments, param-group layout and
state_dict format; the step runs hand-written gfx950 HIP kernels through the C
ABI in include/gefenx.h.
"""
try:  # src/gefen/__init__.py:3-8
    from importlib.metadata import PackageNotFoundError, version

    __version__ = version("gefen-x")
except PackageNotFoundError:
    __version__ = "0.0.0+unknown"

from gefen import kernels
from gefen.gefen import Gefen
from gefen.kernels import period_variance as _period_variance  # noqa: F401 (registers its custom op)
from gefen.gefen_muon import GefenMuon
from gefen.hybrid import GefenMuonHybrid
from gefen.params import DEFAULT_BACKUP_SUBSTRINGS, is_muon_param, split_params_for_muon, validate_split

__all__ = ["Gefen", "GefenMuon", "GefenMuonHybrid", "split_params_for_muon", "validate_split", "is_muon_param",
           "DEFAULT_BACKUP_SUBSTRINGS", "kernels", "__version__"]
