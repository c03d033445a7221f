"""Module-level API: ``PreparedLinear`` replaces ``nn.Linear`` in a model shell.

Mirrors the reference's module binding (src/nanoquant/runtime/torch_model.py:18-90,
684-783): a ``ContextVar`` selects the prefill or decode workload for a whole
forward, the module runs its layer through ``PreparedModel.linear`` and by
default casts the backend's fp32 output back to the input dtype.
"""

from __future__ import annotations

import weakref
from collections.abc import Iterator, Mapping
from contextlib import contextmanager
from contextvars import ContextVar
from typing import Literal

import torch
from torch import nn

from nanoquant_amd.runtime.backend import WorkloadKind
from nanoquant_amd.runtime.dispatch import PreparedModel

_ACTIVE_WORKLOAD: ContextVar[WorkloadKind | None] = ContextVar(
    "nanoquant_amd_active_workload", default=None
)


@contextmanager
def execution_workload(kind: WorkloadKind) -> Iterator[None]:
    """Select the prepared plan used by every ``PreparedLinear`` inside the block
    (src/nanoquant/runtime/torch_model.py:21-31)."""

    if kind not in ("prefill", "decode"):
        raise ValueError(f"unsupported runtime execution workload: {kind}")
    token = _ACTIVE_WORKLOAD.set(kind)
    try:
        yield
    finally:
        _ACTIVE_WORKLOAD.reset(token)


class PreparedLinear(nn.Module):
    """Parameter-free module over one planned layer (src/nanoquant/runtime/torch_model.py:34-66)."""

    def __init__(
        self,
        model: PreparedModel,
        layer_index: int,
        *,
        output_dtype: Literal["input", "backend"] = "input",
    ) -> None:
        super().__init__()
        if output_dtype not in ("input", "backend"):
            raise ValueError(f"unsupported prepared linear output dtype policy: {output_dtype}")
        spec = model.spec(layer_index)
        self._model = model
        self._layer_index = layer_index
        self._output_dtype = output_dtype
        self.in_features = spec.in_features
        self.out_features = spec.out_features

    def forward(self, value: torch.Tensor) -> torch.Tensor:
        kind = _ACTIVE_WORKLOAD.get()
        if kind is None:
            raise RuntimeError(
                "NanoQuant prepared linear executed outside an execution_workload context"
            )
        output = self._model.linear(kind, self._layer_index, value)
        if self._output_dtype == "input":
            return output.to(dtype=value.dtype)
        return output


class PreparedProjectionView(nn.Module):
    """Row slice of a grouped owner's output (src/nanoquant/runtime/torch_model.py:69-90)."""

    def __init__(self, owner: PreparedLinear, row_start: int, row_end: int) -> None:
        super().__init__()
        # A weak reference keeps the owner out of this module's children.
        self.__dict__["_owner_ref"] = weakref.ref(owner)
        self.row_start = row_start
        self.row_end = row_end
        self.in_features = owner.in_features
        self.out_features = row_end - row_start

    def forward(self, value: torch.Tensor) -> torch.Tensor:
        owner = self.__dict__["_owner_ref"]()
        if owner is None:
            raise RuntimeError("prepared shared-input projection owner was released")
        return owner(value)[..., self.row_start : self.row_end]


def transformers_decoder_module_paths(layer_names: tuple[str, ...]) -> dict[str, str]:
    """``blocks.N.rel`` -> ``model.layers.N.rel`` (src/nanoquant/runtime/torch_model.py:771-783)."""

    paths: dict[str, str] = {}
    for name in layer_names:
        head, _, rest = name.partition(".")
        if head != "blocks" or not rest:
            raise ValueError(f"canonical runtime layer is not block-scoped: {name}")
        index, _, relative = rest.partition(".")
        if not index.isdigit() or not relative:
            raise ValueError(f"canonical runtime layer path is invalid: {name}")
        paths[name] = f"model.layers.{index}.{relative}"
    return paths


def _resolve_linear(model: nn.Module, path: str, layer_name: str) -> tuple[nn.Module, str, nn.Module]:
    parent_path, dot, attribute = path.rpartition(".")
    if not dot or not parent_path or not attribute:
        raise ValueError(f"runtime model module path must be dotted: {path!r}")
    try:
        parent = model.get_submodule(parent_path)
        existing = getattr(parent, attribute)
    except (AttributeError, KeyError) as error:
        raise ValueError(f"runtime model module is unavailable for {layer_name}: {path}") from error
    if not isinstance(existing, nn.Linear):
        raise ValueError(f"runtime model target is not a linear module for {layer_name}: {path}")
    return parent, attribute, existing


def bind_prepared_linears(
    model: nn.Module,
    prepared: PreparedModel,
    module_paths: Mapping[str, str],
    *,
    output_dtype: Literal["input", "backend"] = "input",
) -> int:
    """Replace exactly the planned ``nn.Linear`` inventory; validate everything
    before mutating the model (src/nanoquant/runtime/torch_model.py:684-768)."""

    names = prepared.names
    if set(module_paths) != set(names):
        raise ValueError(
            "runtime model module mapping differs from the plan: "
            f"missing={sorted(set(names) - set(module_paths))}, "
            f"unexpected={sorted(set(module_paths) - set(names))}"
        )
    paths = [module_paths[name] for name in names]
    if len(set(paths)) != len(paths):
        raise ValueError("runtime model module paths must be unique")

    swaps: list[tuple[nn.Module, str, nn.Module]] = []
    owners: list[tuple[nn.Module, str, PreparedLinear]] = []
    for index, (name, path) in enumerate(zip(names, paths, strict=True)):
        spec = prepared.spec(index)
        if not spec.members:
            parent, attribute, existing = _resolve_linear(model, path, name)
            if (existing.in_features, existing.out_features) != (spec.in_features, spec.out_features):
                raise ValueError(f"runtime model linear dimensions differ for {name}: {path}")
            swaps.append((parent, attribute, PreparedLinear(prepared, index, output_dtype=output_dtype)))
            continue
        block_path, marker, relative = path.partition(".self_attn.")
        if not (marker and block_path and relative):
            raise ValueError(f"runtime projection group path is invalid for {name}: {path}")
        try:
            block = model.get_submodule(block_path)
        except (AttributeError, KeyError) as error:
            raise ValueError(f"runtime projection group block is unavailable for {name}: {path}") from error
        owner = PreparedLinear(prepared, index, output_dtype=output_dtype)
        for member in spec.members:
            member_path = transformers_decoder_module_paths((member.name,))[member.name]
            parent, attribute, existing = _resolve_linear(model, member_path, name)
            rows = member.row_end - member.row_start
            if (existing.in_features, existing.out_features) != (spec.in_features, rows):
                raise ValueError(
                    f"runtime projection member dimensions differ for {name}: {member_path}"
                )
            swaps.append(
                (parent, attribute, PreparedProjectionView(owner, member.row_start, member.row_end))
            )
        owners.append((block, relative.replace(".", "__"), owner))

    for block, key, owner in owners:
        registry = getattr(block, "_nanoquant_shared_input_groups", None)
        if registry is None:
            registry = nn.ModuleDict()
            block.add_module("_nanoquant_shared_input_groups", registry)
        if not isinstance(registry, nn.ModuleDict) or key in registry:
            raise ValueError("runtime projection group owner registry conflicts with the model")
        registry[key] = owner
    for parent, attribute, replacement in swaps:
        setattr(parent, attribute, replacement)
    return len(names)
