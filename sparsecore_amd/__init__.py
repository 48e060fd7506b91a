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
from . import _lib, nn, ops, router

__all__ = ["PaddedCSR", "spmm", "SparseLinear", "layout", "SparsityAlgorithm", "Static",
           "DynamicSparsityAlgorithm", "SET", "RigL", "install_as_sparselab"]
__version__ = "0.1.0"


def native_available() -> bool:
    """True when the gfx950 library is built and loadable."""
    return _lib.available()


# The reference's module names (sparselab/__init__.py:56-76 and its
# submodules) mapped onto this package's, for install_as_sparselab().
_SPARSELAB_MODULES = ("layout", "ops", "nn", "router")


def install_as_sparselab(force: bool = False) -> None:
    """Make ``import sparselab`` (and ``sparselab.layout / ops / nn /
    router``) resolve to this package, so code written against the reference
    runs on the GPU unchanged. The reference's whole Python layer is replaced,
    not only its ``_core`` extension: its ops.py converts X, dY and dX through
    numpy (ops.py:163-164, :189, :202) and rejects tensors off the CPU
    (:284-288), and its layout.py builds the pybind PaddedCSR from Python
    lists (layout.py:157, :527). Raises RuntimeError if another ``sparselab``
    is already imported, unless ``force``."""
    import sys

    pkg = sys.modules[__name__]
    have = sys.modules.get("sparselab")
    if have is not None and have is not pkg and not force:
        raise RuntimeError(f"install_as_sparselab: a different sparselab is already imported "
                           f"({getattr(have, '__file__', have)!r}); pass force=True to replace it")
    sys.modules["sparselab"] = pkg
    for name in _SPARSELAB_MODULES:
        sys.modules[f"sparselab.{name}"] = sys.modules[f"{__name__}.{name}"]
