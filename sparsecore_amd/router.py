"""sparsecore_amd.router — sparsity policies (Static, SET, RigL) on the device.

Same user surface as ``sparselab/router.py``: ``model.apply(algo)`` attaches
an algorithm to every SparseLinear, ``algo.step()`` after ``opt.step()``
advances the schedule and fires ``update()`` every ``update_freq`` steps.

What differs is where the update runs. The reference walks every row in
Python with numpy (router.py:378-478, :598-732); here one ``update()`` of a
layer is a handful of kernel launches with no host round trip:

    threshold  k-th smallest |v| over live slots      slk_live_abs_kth
    RigL G     dense dY·Xᵀ from the captured tensors    slk_dense_grad (token-major)
    rows       keep / drop / grow / sorted rewrite      slk_drop_grow

Results: the drop set is exactly the reference's (same threshold, same
strict comparison, same "keep the first largest" rule for rows that would
empty). RigL grows the reference's top-|G| columns (ties, which numpy's
argpartition leaves unspecified, go to the lower column). SET grows a
uniform random subset of the row's empty columns, as the reference does, but
from its own counter-based generator (splitmix64 keys) seeded from the
algorithm's ``seed``: the reference's numpy ``Generator.choice`` stream
cannot be reproduced on the device, so SET topologies match the reference's
in distribution, not draw for draw. A row regrows as many columns as it
dropped, except under RigL's NaN rule: a column whose G is NaN is never
grown, so a row with fewer non-NaN empty columns than drops ends shorter
(its capacity is unchanged). Every update bumps the topology version, and
every cached schedule (row order, segment list, phase bounds, binned stream,
the transpose) is keyed by it, so each rebuilds on its next use; only the
longest-first row order is carried over, when no row shrank.
"""

from __future__ import annotations

import numpy as np
import torch

from . import _lib

__all__ = ["SparsityAlgorithm", "DynamicSparsityAlgorithm", "Static", "SET", "RigL"]


class SparsityAlgorithm:
    """Base class of every sparsity policy (router.py:61-171).

    Tracks the attached layers (``self.layers``) and a step counter;
    ``__call__(module)`` attaches SparseLinear modules so that
    ``model.apply(algo)`` works.
    """

    def __init__(self, sparsity: float):
        if not (0.0 <= sparsity < 1.0):
            raise ValueError(f"sparsity must be in [0.0, 1.0), got {sparsity}")
        self.sparsity = sparsity
        self.layers: list = []
        self._step_idx: int = 0

    def attach(self, layer) -> None:
        from .nn import SparseLinear

        if not isinstance(layer, SparseLinear):
            raise TypeError(f"SparsityAlgorithm.attach expects a SparseLinear, "
                            f"got {type(layer).__name__}")
        if layer not in self.layers:
            self.layers.append(layer)
            layer._sparsity_algorithm = self

    def __call__(self, module) -> None:
        from .nn import SparseLinear

        if isinstance(module, SparseLinear):
            self.attach(module)

    def step(self) -> None:
        self._step_idx += 1

    def update(self) -> None:  # pragma: no cover - subclasses override
        raise NotImplementedError("SparsityAlgorithm.update() must be overridden by subclasses")

    def __repr__(self) -> str:
        return (f"{type(self).__name__}(sparsity={self.sparsity}, "
                f"n_layers={len(self.layers)}, step={self._step_idx})")


class Static(SparsityAlgorithm):
    """Keeps the initial mask for the whole run (router.py:179-218)."""

    def update(self) -> None:
        pass


class DynamicSparsityAlgorithm(SparsityAlgorithm):
    """Base of schedule-driven topology updates (router.py:225-289).

    ``step()`` calls ``update()`` whenever the step count is a multiple of
    ``update_freq``.
    """

    def __init__(self, sparsity: float, drop_fraction: float, update_freq: int):
        super().__init__(sparsity=sparsity)
        if not (0.0 < drop_fraction <= 1.0):
            raise ValueError(f"drop_fraction must be in (0.0, 1.0], got {drop_fraction}")
        if update_freq < 1:
            raise ValueError(f"update_freq must be >= 1, got {update_freq}")
        self.drop_fraction = drop_fraction
        self.update_freq = update_freq

    def step(self) -> None:
        self._step_idx += 1
        if self._step_idx % self.update_freq == 0:
            self.update()

    def _rebuild_transposes(self) -> None:
        """After a rewrite, rebuild the cached transposes of the rewritten
        layers in one batch, so the next backward finds them current instead
        of rebuilding each with its own device->host read."""
        from .ops import _rebuild_stale_transposes

        _rebuild_stale_transposes([layer._csr for layer in self.layers])

    def _k_drop(self, total_nnz: int) -> int:
        # Python float product then int(), as router.py:409
        return max(1, int(self.drop_fraction * total_nnz))

    def __repr__(self) -> str:
        return (f"{type(self).__name__}(sparsity={self.sparsity}, "
                f"drop_fraction={self.drop_fraction}, update_freq={self.update_freq}, "
                f"n_layers={len(self.layers)}, step={self._step_idx})")


class SET(DynamicSparsityAlgorithm):
    """Sparse Evolutionary Training (router.py:296-482).

    Each update drops, per layer, every live weight with |w| at or below the
    layer's k-th smallest magnitude (k = max(1, int(drop_fraction·nnz))),
    keeping at least the largest weight of each row, then regrows as many
    connections per row at uniformly random empty columns, initialised to 0.
    ``seed`` makes the sequence of updates reproducible.
    """

    def __init__(self, sparsity: float, drop_fraction: float = 0.3, update_freq: int = 100,
                 seed: int | None = None):
        super().__init__(sparsity=sparsity, drop_fraction=drop_fraction,
                         update_freq=update_freq)
        self._rng = np.random.default_rng(seed)

    def update(self) -> None:
        for layer in self.layers:
            self._update_layer(layer, self._rng)
        self._rebuild_transposes()

    def _update_layer(self, layer, rng) -> None:
        csr = layer._csr
        total_nnz = int(csr.nnz)
        if total_nnz == 0:
            return
        seed = int(rng.integers(0, 2**63, dtype=np.int64))
        csr._drop_grow(self._k_drop(total_nnz), _lib.SLK_GROW_RANDOM, None, seed)


class RigL(DynamicSparsityAlgorithm):
    """Rigging the Lottery (router.py:489-735).

    Same drop rule as SET; grows each row at the empty columns with the
    largest |dL/dW| of the dense gradient G = dYᵀ·X computed from the layer
    input and output gradient of the most recent forward/backward (captured
    by hooks installed at attach time, cleared after each update).
    """

    def __init__(self, sparsity: float, drop_fraction: float = 0.3, update_freq: int = 100,
                 seed: int | None = None):
        super().__init__(sparsity=sparsity, drop_fraction=drop_fraction,
                         update_freq=update_freq)
        self._rng = np.random.default_rng(seed)
        self._captured: dict[int, dict] = {}
        self._hook_handles: list = []

    def attach(self, layer) -> None:
        super().attach(layer)

        def _fwd_hook(mod, inputs, output):
            self._captured.setdefault(id(mod), {})["X"] = inputs[0].detach().clone()

        def _bwd_hook(mod, grad_input, grad_output):
            dY = grad_output[0]
            if dY is not None:
                self._captured.setdefault(id(mod), {})["dY"] = dY.detach().clone()

        self._hook_handles.append(layer.register_forward_hook(_fwd_hook))
        self._hook_handles.append(layer.register_full_backward_hook(_bwd_hook))

    def update(self) -> None:
        for layer in self.layers:
            self._update_layer(layer, self._rng)
        self._rebuild_transposes()

    def _update_layer(self, layer, rng) -> None:
        from .ops import _as_row_major

        captured = self._captured.get(id(layer))
        if captured is None or "X" not in captured or "dY" not in captured:
            return  # no forward/backward since the last update
        csr = layer._csr
        total_nnz = int(csr.nnz)
        if total_nnz == 0:
            self._captured.pop(id(layer), None)
            return
        dev = csr.device
        x = captured["X"].reshape(-1, layer.in_features).to(dev)
        dy = captured["dY"].reshape(-1, layer.out_features).to(dev)
        # grows ranked by |G|, G = dyᵀ·x = (out, in): certified from the
        # matrix-core approximation, exact where it cannot decide
        csr._rigl_update(self._k_drop(total_nnz), _as_row_major(dy.t()), _as_row_major(x.t()))
        self._captured.pop(id(layer), None)
