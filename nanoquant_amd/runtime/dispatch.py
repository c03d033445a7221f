"""Backend selection and prepared layers for one layer inventory.

Callers of the reference runtime keep its own planner
(src/nanoquant/runtime/planning.py:70-299) and list ``HipPackedBackend`` among
its backends; nothing here is needed for that. This module is the package's
standalone route from layer states to prepared layers:

* ``choose_backends`` asks each backend, in priority order, whether it
  ``supports`` a layer under one workload and keeps the first that does,
  together with every earlier backend's stable rejection code;
* ``PreparedModel`` makes that choice for a prefill and a decode workload,
  prepares each (layer, backend) pair once (both workloads share the device
  payload when they chose the same backend) and runs a layer after checking
  the input against the workload it was chosen for.
"""

from __future__ import annotations

from collections.abc import Mapping, Sequence
from dataclasses import dataclass
from math import prod

import torch

from nanoquant_amd.runtime.backend import (
    DeviceLike,
    PreparedLayer,
    QuantizedLinearSpec,
    RuntimeBackend,
    RuntimeLayerState,
    WorkloadKind,
    WorkloadSpec,
)
from nanoquant_amd.runtime.logical import canonical_torch_dtype


class SelectionError(RuntimeError):
    """No backend accepted a layer, or a strict selection needed a fallback."""


@dataclass(frozen=True, slots=True)
class Rejection:
    """One backend's answer for one layer: ``backend`` is ``name@version``."""

    backend: str
    code: str
    reason: str


@dataclass(frozen=True, slots=True)
class Choice:
    """The backend chosen for one layer and the backends tried before it."""

    layer: str
    backend: RuntimeBackend
    rejections: tuple[Rejection, ...]

    @property
    def fallback(self) -> bool:
        return bool(self.rejections)


def _tag(backend: RuntimeBackend) -> str:
    return f"{backend.name}@{backend.version}"


def choose_backends(
    specs: Sequence[QuantizedLinearSpec],
    workload: WorkloadSpec,
    backends: Sequence[RuntimeBackend],
    *,
    strict: bool,
) -> tuple[Choice, ...]:
    """First supporting backend per layer. ``strict`` refuses any layer whose
    first-priority backend declined it."""

    names = [spec.name for spec in specs]
    if not names:
        raise ValueError("backend selection needs at least one layer")
    if len(set(names)) != len(names):
        raise ValueError("layer names must be unique")
    tags = [_tag(b) for b in backends]
    if not tags:
        raise ValueError("backend selection needs at least one backend")
    if len(set(tags)) != len(tags):
        raise ValueError("backends must differ in name or version")
    choices = []
    for spec in specs:
        tried: list[Rejection] = []
        for backend in backends:
            answer = backend.supports(spec, workload)
            if answer.supported:
                break
            tried.append(Rejection(_tag(backend), str(answer.code), answer.reason))
        else:
            listing = "; ".join(f"{r.backend} {r.code} ({r.reason})" for r in tried)
            raise SelectionError(f"{spec.name}: no backend accepts the {workload.kind} workload: {listing}")
        if strict and tried:
            first = tried[0]
            raise SelectionError(
                f"{spec.name}: strict selection refuses the fallback to {_tag(backend)} "
                f"after {first.backend} {first.code} ({first.reason})"
            )
        choices.append(Choice(spec.name, backend, tuple(tried)))
    return tuple(choices)


class PreparedModel:
    """Prepared layers of one inventory for a prefill and a decode workload.

    ``states`` maps layer names to layer states; the inventory order is the
    mapping's order. The decode workload must be one token per batch item and
    both workloads must name the device type of ``device``."""

    def __init__(
        self,
        states: Mapping[str, RuntimeLayerState],
        *,
        prefill: WorkloadSpec,
        decode: WorkloadSpec,
        backends: Sequence[RuntimeBackend],
        device: DeviceLike,
        strict: bool = True,
        decode_backends: Sequence[RuntimeBackend] | None = None,
    ) -> None:
        if (prefill.kind, decode.kind) != ("prefill", "decode"):
            raise ValueError("PreparedModel takes a prefill and a decode workload")
        if decode.token_count != 1:
            raise ValueError("the decode workload runs one token per batch item")
        target = torch.device(device)
        for workload in (prefill, decode):
            if workload.device_type != target.type:
                raise ValueError(
                    f"{workload.kind} workload device {workload.device_type!r} is not the "
                    f"preparation device {target.type!r}"
                )
        for name, state in states.items():
            if state.spec.name != name:
                raise ValueError(f"layer state {state.spec.name!r} is stored under the name {name!r}")
        specs = [state.spec for state in states.values()]
        self.names = tuple(states)
        self._workloads = {"prefill": prefill, "decode": decode}
        self._choices = {
            "prefill": choose_backends(specs, prefill, backends, strict=strict),
            "decode": choose_backends(specs, decode, decode_backends or backends, strict=strict),
        }
        made: dict[tuple[str, str], PreparedLayer] = {}
        self._layers: dict[str, tuple[PreparedLayer, ...]] = {}
        for kind, choices in self._choices.items():
            row = []
            for choice in choices:
                key = (choice.layer, _tag(choice.backend))
                if key not in made:
                    layer = choice.backend.prepare(states[choice.layer], target)
                    if layer.spec != states[choice.layer].spec:
                        raise ValueError(f"{choice.layer}: the prepared layer's spec differs from its state")
                    made[key] = layer
                row.append(made[key])
            self._layers[kind] = tuple(row)

    def workload(self, kind: WorkloadKind) -> WorkloadSpec:
        return self._workloads[kind]

    def choices(self, kind: WorkloadKind) -> tuple[Choice, ...]:
        return self._choices[kind]

    def prepared(self, kind: WorkloadKind, index: int) -> PreparedLayer:
        return self._layers[kind][index]

    def spec(self, index: int) -> QuantizedLinearSpec:
        return self._layers["prefill"][index].spec

    def index(self, name: str) -> int:
        return self.names.index(name)

    def linear(self, kind: WorkloadKind, index: int, value: torch.Tensor) -> torch.Tensor:
        """Run layer ``index`` with the backend chosen for ``kind``. The input must
        match that workload: device type, dtype, feature width, batch size and
        token slots (exactly batch x tokens for decode, at most that for prefill)."""

        if kind not in self._workloads:
            raise ValueError(f"unknown workload kind {kind!r}")
        if not 0 <= index < len(self.names):
            raise IndexError(f"layer index {index} is not in the inventory of {len(self.names)}")
        work = self._workloads[kind]
        layer = self._layers[kind][index]
        name = self.names[index]
        if value.device.type != work.device_type:
            raise ValueError(f"{name}: {kind} input is on {value.device.type!r}, not {work.device_type!r}")
        if canonical_torch_dtype(value.dtype) != work.input_dtype:
            raise ValueError(f"{name}: {kind} input dtype {value.dtype} is not {work.input_dtype}")
        if value.ndim < 2 or value.shape[-1] != layer.spec.in_features:
            raise ValueError(f"{name}: {kind} input width is not {layer.spec.in_features}")
        if value.shape[0] != work.batch_size:
            raise ValueError(f"{name}: {kind} batch {value.shape[0]} is not {work.batch_size}")
        limit = work.batch_size * work.token_count
        slots = prod(value.shape[:-1])
        if kind == "decode" and slots != limit:
            raise ValueError(f"{name}: decode input holds {slots} token slots; it must hold {limit}")
        if not 0 < slots <= limit:
            raise ValueError(f"{name}: prefill input holds {slots} token slots; at most {limit} fit")
        return self._choices[kind][index].backend.linear(value, layer)
