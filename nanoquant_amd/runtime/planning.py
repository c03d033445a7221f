"""Ahead-of-inference backend planning with explicit fallback reporting.

Mirrors the reference planner (src/nanoquant/runtime/planning.py:23-299): one
backend is resolved per layer before the token loop, strict plans refuse
fallback, paired prefill/decode plans share prepared payloads, and the hot
``linear_at`` checks the planned geometry before calling the backend.
"""

from __future__ import annotations

from collections.abc import Mapping
from dataclasses import dataclass
from math import prod

import torch

from nanoquant_amd.runtime.backend import (
    DeviceLike,
    PreparedLayer,
    QuantizedLinearSpec,
    RuntimeBackend,
    RuntimeLayerState,
    SupportResult,
    WorkloadSpec,
)
from nanoquant_amd.runtime.logical import canonical_torch_dtype


@dataclass(frozen=True, slots=True)
class BackendRejection:
    backend_name: str
    backend_version: str
    support: SupportResult


@dataclass(frozen=True, slots=True)
class LayerDispatch:
    layer_name: str
    backend_name: str
    backend_version: str
    fallback: bool
    rejected_backends: tuple[BackendRejection, ...]


@dataclass(frozen=True, slots=True)
class BackendPlan:
    workload: WorkloadSpec
    layers: tuple[LayerDispatch, ...]
    fallback_count: int


@dataclass(frozen=True, slots=True)
class ExecutionPlans:
    """Independently selected prefill and decode plans over one layer inventory
    (src/nanoquant/runtime/planning.py:46-63)."""

    prefill: BackendPlan
    decode: BackendPlan

    def __post_init__(self) -> None:
        if (self.prefill.workload.kind, self.decode.workload.kind) != ("prefill", "decode"):
            raise ValueError("runtime execution plans require prefill and decode workloads")
        if self.decode.workload.token_count != 1:
            raise ValueError("runtime decode plans require exactly one token per batch item")
        if self.prefill.workload.device_type != self.decode.workload.device_type:
            raise ValueError("runtime prefill and decode plans must use the same device type")
        prefill_names = [entry.layer_name for entry in self.prefill.layers]
        decode_names = [entry.layer_name for entry in self.decode.layers]
        if prefill_names != decode_names:
            raise ValueError("runtime prefill and decode plan layer inventories differ")


class BackendPlanningError(RuntimeError):
    pass


def _backend_key(backend: RuntimeBackend) -> tuple[str, str]:
    return (backend.name, backend.version)


def plan_backends(
    layers: tuple[QuantizedLinearSpec, ...],
    workload: WorkloadSpec,
    backends: tuple[RuntimeBackend, ...],
    *,
    strict: bool,
) -> BackendPlan:
    """Pick the first supporting backend per layer, recording every rejection
    (src/nanoquant/runtime/planning.py:70-114)."""

    if not layers:
        raise ValueError("runtime backend planning requires at least one layer")
    if len({layer.name for layer in layers}) != len(layers):
        raise ValueError("runtime backend planning layer names must be unique")
    if not backends:
        raise ValueError("runtime backend planning requires at least one backend")
    keys = [_backend_key(backend) for backend in backends]
    if len(set(keys)) != len(keys):
        raise ValueError("runtime backend names and versions must be unique")

    dispatches: list[LayerDispatch] = []
    for layer in layers:
        rejections: list[BackendRejection] = []
        chosen: RuntimeBackend | None = None
        for backend in backends:
            answer = backend.supports(layer, workload)
            if answer.supported:
                chosen = backend
                break
            rejections.append(BackendRejection(backend.name, backend.version, answer))
        if chosen is None:
            detail = "; ".join(
                f"{r.backend_name}@{r.backend_version}: {r.support.code} {r.support.reason}"
                for r in rejections
            )
            raise BackendPlanningError(f"no runtime backend supports {layer.name}: {detail}")
        if strict and rejections:
            first = rejections[0]
            raise BackendPlanningError(
                f"strict runtime plan rejected fallback for {layer.name}: "
                f"{first.backend_name}@{first.backend_version} "
                f"{first.support.code} {first.support.reason}"
            )
        dispatches.append(
            LayerDispatch(layer.name, chosen.name, chosen.version, bool(rejections), tuple(rejections))
        )
    return BackendPlan(workload, tuple(dispatches), sum(1 for d in dispatches if d.fallback))


def plan_execution_workloads(
    layers: tuple[QuantizedLinearSpec, ...],
    *,
    prefill: WorkloadSpec,
    decode: WorkloadSpec,
    prefill_backends: tuple[RuntimeBackend, ...],
    decode_backends: tuple[RuntimeBackend, ...],
    strict: bool,
) -> ExecutionPlans:
    """Resolve prefill and decode independently in one layer order
    (src/nanoquant/runtime/planning.py:117-135)."""

    if prefill.kind != "prefill":
        raise ValueError("runtime prefill plan requires a prefill workload")
    if decode.kind != "decode":
        raise ValueError("runtime decode plan requires a decode workload")
    return ExecutionPlans(
        plan_backends(layers, prefill, prefill_backends, strict=strict),
        plan_backends(layers, decode, decode_backends, strict=strict),
    )


@dataclass(frozen=True, slots=True)
class PreparedDispatch:
    plan: LayerDispatch
    backend: RuntimeBackend
    layer: PreparedLayer

    def linear(self, value: torch.Tensor) -> torch.Tensor:
        return self.backend.linear(value, self.layer)


@dataclass(frozen=True, slots=True)
class PreparedBackendPlan:
    plan: BackendPlan
    dispatches: tuple[PreparedDispatch, ...]

    def __post_init__(self) -> None:
        if len(self.plan.layers) != len(self.dispatches):
            raise ValueError("prepared runtime dispatch count differs from its plan")
        if any(d.plan != p for p, d in zip(self.plan.layers, self.dispatches, strict=True)):
            raise ValueError("prepared runtime dispatch order differs from its plan")

    def linear_at(self, layer_index: int, value: torch.Tensor) -> torch.Tensor:
        """Run one planned layer after checking device, dtype, features and slots
        (src/nanoquant/runtime/planning.py:160-200)."""

        if not 0 <= layer_index < len(self.dispatches):
            raise IndexError(f"runtime plan layer index is outside the inventory: {layer_index}")
        dispatch = self.dispatches[layer_index]
        workload = self.plan.workload
        kind = workload.kind
        if value.device.type != workload.device_type:
            raise ValueError(
                f"runtime {kind} input device {value.device.type!r} differs from "
                f"planned device {workload.device_type!r}"
            )
        if canonical_torch_dtype(value.dtype) != workload.input_dtype:
            raise ValueError(
                f"runtime {kind} input dtype differs from planned dtype {workload.input_dtype!r}"
            )
        if value.ndim < 2 or value.shape[-1] != dispatch.layer.spec.in_features:
            raise ValueError(
                f"runtime {kind} input feature dimension differs for {dispatch.plan.layer_name}"
            )
        if value.shape[0] != workload.batch_size:
            raise ValueError(
                f"runtime {kind} input batch size {value.shape[0]} differs from "
                f"planned batch size {workload.batch_size}"
            )
        planned_slots = workload.batch_size * workload.token_count
        slots = prod(value.shape[:-1])
        too_many = slots > planned_slots
        wrong_decode = kind == "decode" and slots != planned_slots
        if slots <= 0 or too_many or wrong_decode:
            bound = "exactly" if kind == "decode" else "at most"
            raise ValueError(
                f"runtime {kind} input has {slots} token slots, expected {bound} {planned_slots}"
            )
        return dispatch.linear(value)


@dataclass(frozen=True, slots=True)
class PreparedExecutionPlans:
    prefill: PreparedBackendPlan
    decode: PreparedBackendPlan

    def __post_init__(self) -> None:
        ExecutionPlans(self.prefill.plan, self.decode.plan)


def _check_inventory(plan: BackendPlan, states: Mapping[str, RuntimeLayerState]) -> None:
    planned = {entry.layer_name for entry in plan.layers}
    given = set(states)
    if planned != given:
        raise ValueError(
            "runtime layer state inventory differs from the plan: "
            f"missing={sorted(planned - given)}, unexpected={sorted(given - planned)}"
        )


def _registry(backends: tuple[RuntimeBackend, ...]) -> dict[tuple[str, str], RuntimeBackend]:
    table = {_backend_key(backend): backend for backend in backends}
    if len(table) != len(backends):
        raise ValueError("runtime backend names and versions must be unique")
    return table


def _prepare_dispatches(
    plan: BackendPlan,
    states: Mapping[str, RuntimeLayerState],
    registry: Mapping[tuple[str, str], RuntimeBackend],
    device: DeviceLike,
    cache: dict[tuple[str, str, str], PreparedLayer],
) -> tuple[PreparedDispatch, ...]:
    prepared: list[PreparedDispatch] = []
    for entry in plan.layers:
        key = (entry.backend_name, entry.backend_version)
        backend = registry.get(key)
        if backend is None:
            raise ValueError(
                f"planned runtime backend is unavailable: {entry.backend_name}@{entry.backend_version}"
            )
        state = states[entry.layer_name]
        if state.spec.name != entry.layer_name:
            raise ValueError(
                f"runtime layer state name differs from its plan entry: {entry.layer_name}"
            )
        cache_key = (entry.layer_name, *key)
        layer = cache.get(cache_key)
        if layer is None:
            layer = backend.prepare(state, device)
            if layer.spec != state.spec or (layer.backend_name, layer.backend_version) != key:
                raise ValueError(f"runtime backend prepared an inconsistent layer: {entry.layer_name}")
            cache[cache_key] = layer
        prepared.append(PreparedDispatch(entry, backend, layer))
    return tuple(prepared)


def prepare_plan(
    plan: BackendPlan,
    states: Mapping[str, RuntimeLayerState],
    backends: tuple[RuntimeBackend, ...],
    device: DeviceLike,
) -> tuple[PreparedDispatch, ...]:
    """Prepare one plan (src/nanoquant/runtime/planning.py:263-270)."""

    _check_inventory(plan, states)
    return _prepare_dispatches(plan, states, _registry(backends), device, {})


def prepare_execution_workloads(
    plans: ExecutionPlans,
    states: Mapping[str, RuntimeLayerState],
    backends: tuple[RuntimeBackend, ...],
    device: DeviceLike,
) -> PreparedExecutionPlans:
    """Prepare both plans, preparing each (layer, backend, version) once
    (src/nanoquant/runtime/planning.py:273-299)."""

    target = torch.device(device)
    planned_type = plans.prefill.workload.device_type
    if target.type != planned_type:
        raise ValueError(
            f"runtime preparation device {target.type!r} differs from planned device {planned_type!r}"
        )
    _check_inventory(plans.prefill, states)
    _check_inventory(plans.decode, states)
    registry = _registry(backends)
    shared: dict[tuple[str, str, str], PreparedLayer] = {}
    return PreparedExecutionPlans(
        PreparedBackendPlan(
            plans.prefill, _prepare_dispatches(plans.prefill, states, registry, device, shared)
        ),
        PreparedBackendPlan(
            plans.decode, _prepare_dispatches(plans.decode, states, registry, device, shared)
        ),
    )
