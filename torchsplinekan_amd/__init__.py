"""torchsplinekan_amd -- B-spline KAN layers with a native MI355X (gfx950) backend.

Drop-in for the torch-spline-kan hot path: ``KANLinear`` / ``KAN`` with the
same API, backed by ``torchsplinekan_amd._C`` (the replacement of
``spline_kan._C``), whose device work runs in libkan_hip.so.
"""

from .kan_linear import KANLinear
from .kan import KAN
from .pruning import PruneResult, prune_nodes

__version__ = "0.1.0"

__all__ = ["KANLinear", "KAN", "PruneResult", "prune_nodes", "__version__"]
