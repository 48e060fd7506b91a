"""sparsecore_amd.nn — ``SparseLinear``, a padded-CSR drop-in for ``nn.Linear``.

Same constructor, attributes (``_csr``, ``_values``, ``bias``), initialisation
and forward as ``sparselab/nn.py:36-268``. The weights live in a PaddedCSR
whose ``values`` tensor *is* the ``_values`` Parameter's storage, so an
optimizer step on ``_values`` is what the next forward reads. Moving the
module (``.cuda()``, ``.to(device)``) moves the CSR with it and keeps that
aliasing; the forward and backward run on the HIP device only.
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn

from . import layout as _layout
from .layout import PaddedCSR
from . import ops as _ops
from .ops import _SparseLinearFunction

__all__ = ["SparseLinear"]


class SparseLinear(nn.Module):
    """Linear layer whose weight is a PaddedCSR at the requested sparsity.

    Args:
        in_features, out_features: layer sizes.
        bias: learn an additive bias (default True).
        sparsity: fraction of structurally-zero weights, in [0, 1) (default 0.9).
        padding_ratio: spare capacity per row for topology updates (default 0.2).
        device: where to place the layer (default: CPU, as torch layers do;
            move it to the GPU with ``.cuda()`` before running it).

    Shape: input (*, in_features) -> output (*, out_features).
    """

    def __init__(self, in_features: int, out_features: int, bias: bool = True,
                 sparsity: float = 0.9, padding_ratio: float = 0.2, device=None):
        super().__init__()
        if not (0.0 <= sparsity < 1.0):
            raise ValueError(f"sparsity must be in [0.0, 1.0), got {sparsity}")
        self.in_features = in_features
        self.out_features = out_features
        self.sparsity = sparsity
        self.padding_ratio = padding_ratio
        self._csr, values_param = self._build_csr_and_parameter(sparsity)
        self._values = values_param
        if bias:
            self.bias = nn.Parameter(torch.empty(out_features))
        else:
            self.register_parameter("bias", None)
        if self.bias is not None:
            effective_fan_in = max(1.0, in_features * (1.0 - sparsity))
            bound = 1.0 / math.sqrt(effective_fan_in)
            nn.init.uniform_(self.bias, -bound, bound)
        if device is not None:
            self.to(device)

    def _build_csr_and_parameter(self, sparsity: float) -> tuple[PaddedCSR, nn.Parameter]:
        """Fresh mask + values (nn.py:118-185, same torch RNG order), aliased Parameter."""
        effective_fan_in = max(1.0, self.in_features * (1.0 - sparsity))
        bound = 1.0 / math.sqrt(effective_fan_in)
        W_dense = torch.empty(self.out_features, self.in_features)
        nn.init.uniform_(W_dense, -bound, bound)
        mask = torch.rand(self.out_features, self.in_features) >= sparsity
        W_dense = W_dense * mask.float()
        csr = _layout.from_dense(W_dense, padding_ratio=self.padding_ratio)
        values_param = nn.Parameter(csr.values)
        csr._bind_values(values_param.data)
        return csr, values_param

    def reset_parameters(self) -> None:
        """Redraw mask, values and bias (nn.py:187-204)."""
        device = self._values.device
        csr, new_values = self._build_csr_and_parameter(self.sparsity)
        csr = csr.to(device)
        with torch.no_grad():
            self._values.data = csr.values
        csr._bind_values(self._values.data)
        self._csr = csr
        if self.bias is not None:
            bound = 1.0 / math.sqrt(self.in_features)
            nn.init.uniform_(self.bias, -bound, bound)

    def _apply(self, fn, *args, **kwargs):
        """Keep the CSR on the values' device and aliased with ``_values``."""
        out = super()._apply(fn, *args, **kwargs)
        v = self._values.data
        if self._csr.device != v.device:
            self._csr = self._csr.to(v.device)
        if v.dtype == torch.float32 and v.is_contiguous():
            self._csr._bind_values(v)
        return out

    # ─── topology serialization ────────────────────────────────────────
    # The reference's state_dict holds only the values and the bias, so a
    # receiver has to rebuild the same mask from the same seed
    # (tests/test_sparse_linear.py:312-335). Here the topology travels too:
    # the four structure arrays and the topology version are saved next to
    # ``_values``, and loading them installs that topology (validated by the
    # invariant checker) before the values are copied. A state dict without
    # them — a reference-style checkpoint — loads values only, as before.
    _TOPOLOGY_KEYS = ("csr_col_indices", "csr_row_start", "csr_row_nnz", "csr_row_capacity",
                      "csr_topology_version")

    def _save_to_state_dict(self, destination, prefix, keep_vars):
        super()._save_to_state_dict(destination, prefix, keep_vars)
        csr = self._csr
        destination[prefix + "csr_col_indices"] = csr.col_indices.detach()
        destination[prefix + "csr_row_start"] = csr.row_start.detach()
        destination[prefix + "csr_row_nnz"] = csr.row_nnz.detach()
        destination[prefix + "csr_row_capacity"] = csr.row_capacity.detach()
        destination[prefix + "csr_topology_version"] = torch.tensor(csr.topology_version,
                                                                    dtype=torch.int64)

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                              unexpected_keys, error_msgs):
        keys = [prefix + k for k in self._TOPOLOGY_KEYS]
        present = [k in state_dict for k in keys]
        if any(present) and not all(present):
            error_msgs.append(f"SparseLinear: partial topology in state_dict (need all of "
                              f"{', '.join(keys)})")
        elif all(present) and prefix + "_values" in state_dict:
            vals = state_dict[prefix + "_values"]
            dev = self._values.device
            try:
                csr = PaddedCSR(self.out_features, self.in_features,
                                vals.detach().to(dev, torch.float32),
                                *(state_dict[k].to(dev, torch.int32) for k in keys[:4]),
                                device=dev)
            except ValueError as e:
                error_msgs.append(f"SparseLinear: invalid topology in state_dict: {e}")
            else:
                csr._topology_version = int(state_dict[keys[4]])
                with torch.no_grad():
                    self._values.data = csr.values
                csr._bind_values(self._values.data)
                self._csr = csr
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs)
        for k in keys:
            if k in unexpected_keys:
                unexpected_keys.remove(k)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """y = x @ Wᵀ + b with W stored as PaddedCSR (nn.py:210-245)."""
        orig_shape = x.shape
        if orig_shape[-1] != self.in_features:
            raise ValueError(f"SparseLinear expects input last dim {self.in_features}, "
                             f"got {orig_shape[-1]}")
        # One autograd node: the (N, in) -> (in, N) layout change (none when x
        # is the transposed view a previous SparseLinear returned), the SpMM
        # with the bias add fused into its store, and the matching backward.
        # A narrow layer (few outputs) gets its output token-major and
        # contiguous straight from the store; otherwise the output is the
        # transposed view of the feature-major result.
        x_flat = x.reshape(-1, self.in_features)
        if x_flat.dtype != torch.float32:
            x_flat = x_flat.to(torch.float32)
        narrow = _ops._narrow_layer(self._csr)
        b = self.bias
        if b is not None and b.dtype != torch.float32:
            out = _SparseLinearFunction.apply(self._values, None, self._csr, x_flat, "simd")
            y_flat = (out if narrow else out.t()) + b.to(torch.float32)
        else:
            out = _SparseLinearFunction.apply(self._values, b, self._csr, x_flat, "simd")
            y_flat = out if narrow else out.t()
        return y_flat.reshape(orig_shape[:-1] + (self.out_features,))

    @property
    def nnz(self) -> int:
        return self._csr.nnz

    @property
    def density(self) -> float:
        return self.nnz / (self.out_features * self.in_features)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, sparsity={self.sparsity}, nnz={self.nnz}")
