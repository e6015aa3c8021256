"""MI355X-native dilution attention: the operator hot path of
Royer-Research-Labs/Dilution-Attention on hand-written gfx950 HIP kernels.

`dilution.kernels` is the drop-in for the reference module of the same name.
"""

from . import cache, kernels

__all__ = ["cache", "kernels"]
