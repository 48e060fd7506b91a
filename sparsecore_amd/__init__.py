"""sparsecore_amd — MI355X (gfx950) padded-CSR sparse-training hot path.

A GPU drop-in for the hot path of SparseLab (DarshanFofadiya/sparsecore):

    PaddedCSR      padded-row CSR matrix in device memory      (sparselab.PaddedCSR)
    spmm(W, X)     Y = W @ X, autograd-aware                   (sparselab.spmm)
    SparseLinear   nn.Linear replacement backed by PaddedCSR   (sparselab.SparseLinear)
    Static/SET/RigL  sparsity policies, updates on the device  (sparselab.router)

The kernels (forward SpMM, live-slot dW, device transpose and cache refresh,
invariant scan) are hand-written HIP for gfx950 in ``csrc/``, built into
``_lib/libsparsecore_amd.so`` and reached through the C-ABI declared in
``include/sparsecore_amd.h``. There is no CPU fallback.
"""

import torch as _torch  # noqa: F401  (load torch's HIP runtime before the library)

from . import layout
from .layout import PaddedCSR
from .ops import spmm
from .nn import SparseLinear
from .router import DynamicSparsityAlgorithm, RigL, SET, SparsityAlgorithm, Static
from . import _lib

__all__ = ["PaddedCSR", "spmm", "SparseLinear", "layout", "SparsityAlgorithm", "Static",
           "DynamicSparsityAlgorithm", "SET", "RigL"]
__version__ = "0.1.0"


def native_available() -> bool:
    """True when the gfx950 library is built and loadable."""
    return _lib.available()
