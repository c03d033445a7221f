"""Output-row int8 sidecar: dense int8 rows added to selected *output* rows.

The reference runtime's sidecar indexes input columns (``PackedLayerState``
``outlier_*``). An output-row sidecar has no field there, but it is exactly a
float low-rank patch (src/nanoquant/runtime/reference.py:224-233):

    patch_right[k, :] = float(int8_row_k)
    patch_left[o, k]  = row_scale[k] if o == row_index[k] else 0

``RowSidecarLayerState.to_logical()`` produces that patch, so every torch
reference backend evaluates it; the HIP backend runs the compact int8 form.
"""

from __future__ import annotations

from dataclasses import dataclass, replace

import torch

from nanoquant_amd.runtime.backend import QuantizedLinearSpec
from nanoquant_amd.runtime.logical import LogicalLayerState, canonical_torch_dtype
from nanoquant_amd.runtime.packed import PackedLayerState


@dataclass(frozen=True, slots=True)
class OutputRowSidecar:
    indices: torch.Tensor  # int32 [k], strictly increasing, < out_features
    values: torch.Tensor  # int8 [k, in_features]
    scales: torch.Tensor  # [k], the layer's scale dtype

    def validate(self, spec: QuantizedLinearSpec) -> None:
        k = int(self.indices.numel())
        if self.indices.dtype != torch.int32 or self.indices.ndim != 1 or k == 0:
            raise ValueError("output-row sidecar indices must be a non-empty int32 vector")
        if self.values.dtype != torch.int8 or tuple(self.values.shape) != (k, spec.in_features):
            raise ValueError("output-row sidecar values must be int8 [rows, in_features]")
        if tuple(self.scales.shape) != (k,):
            raise ValueError("output-row sidecar scales must have one value per row")
        if canonical_torch_dtype(self.scales.dtype) != spec.scale_dtype:
            raise ValueError("output-row sidecar scale dtype differs from the scale dtype")
        if not bool(torch.isfinite(self.scales).all()):
            raise ValueError("output-row sidecar scale contains a non-finite value")
        if not all(t.is_contiguous() for t in (self.indices, self.values, self.scales)):
            raise ValueError("output-row sidecar tensors must be contiguous")
        index = self.indices.to(torch.int64)
        if bool((index < 0).any()) or bool((index >= spec.out_features).any()):
            raise ValueError("output-row sidecar index is outside the output dimension")
        if not bool((index[1:] > index[:-1]).all()):
            raise ValueError("output-row sidecar indices must be strictly increasing")


@dataclass(frozen=True, slots=True)
class RowSidecarLayerState:
    """A packed layer plus an output-row int8 sidecar."""

    base: PackedLayerState
    rows: OutputRowSidecar

    def __post_init__(self) -> None:
        if self.base.patch_left is not None:
            raise ValueError("output-row sidecar layers cannot also carry a float patch")
        self.rows.validate(self.base.spec)

    @property
    def spec(self) -> QuantizedLinearSpec:
        return self.base.spec

    def as_patch(self) -> tuple[torch.Tensor, torch.Tensor]:
        """The equivalent float32 (patch_left [out, k], patch_right [k, in])."""

        spec = self.base.spec
        k = int(self.rows.indices.numel())
        left = torch.zeros(spec.out_features, k, dtype=torch.float32)
        left[self.rows.indices.long().cpu(), torch.arange(k)] = self.rows.scales.float().cpu()
        right = self.rows.values.float().cpu().contiguous()
        return left, right

    def to_logical(self) -> LogicalLayerState:
        logical = self.base.to_logical()
        left, right = self.as_patch()
        spec = replace(logical.spec, patch_rank=left.shape[1], patch_value_dtype="float32")
        return LogicalLayerState(
            spec,
            logical.left_binary,
            logical.right_binary,
            logical.scale_pre,
            logical.scale_mid,
            logical.scale_post,
            logical.bias,
            logical.outlier_indices,
            logical.outlier_values,
            logical.outlier_scales,
            left,
            right,
        )
