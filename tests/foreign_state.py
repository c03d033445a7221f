"""Stand-ins for the reference runtime's own dataclasses.

A caller of the reference holds its own ``QuantizedLinearSpec``,
``WorkloadSpec``, ``PackedLayerState`` and ``MixedVLayerState`` objects
(src/nanoquant/runtime/backend.py:27-91, packed.py:231-244,
mixed_v.py:169-187). These classes carry exactly those field names, derive
from nothing in ``nanoquant_amd`` and import nothing from the reference, so a
test can hand the HIP backend objects it has never seen the classes of.
"""

from __future__ import annotations

from dataclasses import dataclass, fields

import torch


@dataclass(frozen=True, slots=True)
class ForeignSpec:
    name: str
    logical_format: str
    in_features: int
    out_features: int
    rank: int
    factor_dtype: str
    scale_dtype: str
    outlier_count: int = 0
    outlier_value_dtype: str | None = None
    has_outlier_scales: bool = False
    has_bias: bool = False
    members: tuple = ()
    patch_rank: int = 0
    patch_value_dtype: str | None = None
    bias_dtype: str | None = None


@dataclass(frozen=True, slots=True)
class ForeignWorkload:
    kind: str
    device_type: str
    input_dtype: str
    batch_size: int
    token_count: int
    deterministic: bool = False


@dataclass(frozen=True, slots=True)
class ForeignPackedLayerState:
    spec: ForeignSpec
    layout: str
    left_words: torch.Tensor
    right_words: torch.Tensor
    scale_pre: torch.Tensor
    scale_mid: torch.Tensor
    scale_post: torch.Tensor
    bias: torch.Tensor | None = None
    outlier_indices: torch.Tensor | None = None
    outlier_values: torch.Tensor | None = None
    outlier_scales: torch.Tensor | None = None
    patch_left: torch.Tensor | None = None
    patch_right: torch.Tensor | None = None


@dataclass(frozen=True, slots=True)
class ForeignMixedVLayerState:
    spec: ForeignSpec
    format: str
    free_rows: int
    left_words: torch.Tensor
    free_right_words: torch.Tensor
    coded_payload: torch.Tensor
    codebook_words: torch.Tensor
    scale_pre: torch.Tensor
    scale_mid: torch.Tensor
    scale_post: torch.Tensor
    bias: torch.Tensor | None = None
    outlier_indices: torch.Tensor | None = None
    outlier_values: torch.Tensor | None = None
    outlier_scales: torch.Tensor | None = None
    patch_left: torch.Tensor | None = None
    patch_right: torch.Tensor | None = None


def foreign_spec(spec) -> ForeignSpec:
    """A ForeignSpec with the same field values as ``spec`` (members kept as is)."""

    return ForeignSpec(**{f.name: getattr(spec, f.name) for f in fields(ForeignSpec)})


def foreign_copy(state, cls=ForeignPackedLayerState):
    """``state``'s fields in a stand-in of class ``cls``, with a ForeignSpec."""

    values = {f.name: getattr(state, f.name, None) for f in fields(cls)}
    values["spec"] = foreign_spec(state.spec)
    return cls(**values)
