"""strata_hip: strata-mlx's decode-step hot path for MI355X (gfx950).

The modules mirror the reference's (strata_mlx/blocks.py, fused.py, attention.py) with the same names, argument
order and return conventions, on torch tensors on the GPU, over hand-written HIP kernels behind a C ABI
(libstrata_hip.so, include/strata_hip.h). There is no CPU path: calls raise when the library is not built.
"""

from . import tables  # noqa: F401
from ._lib import StrataHipError, load  # noqa: F401
