"""Backend contract for the packed binary low-rank linear.

Mirrors the reference runtime's backend protocol so a HIP backend drops into the
same planner: ``QuantizedLinearSpec`` / ``WorkloadSpec`` / ``BackendCapabilities``
/ ``SupportResult`` / ``PreparedLayer`` / ``RuntimeBackend`` and the ordered
capability check with stable ``NQ-INF-*`` codes
(src/nanoquant/runtime/backend.py:14-266).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal, Protocol, TypeAlias, runtime_checkable

import torch

DeviceLike: TypeAlias = str | torch.device
WorkloadKind: TypeAlias = Literal["prefill", "decode"]

_WORKLOAD_KINDS = ("prefill", "decode")


def _canonical_name(name: str) -> bool:
    return bool(name) and not name.startswith("/") and ".." not in name.split(".")


@dataclass(frozen=True, slots=True)
class ProjectionMemberSpec:
    """One member of a grouped projection: rows ``[row_start, row_end)`` of the output
    (src/nanoquant/runtime/backend.py:14-24)."""

    name: str
    row_start: int
    row_end: int

    def __post_init__(self) -> None:
        if not _canonical_name(self.name):
            raise ValueError("runtime projection member name must be canonical")
        if not 0 <= self.row_start < self.row_end:
            raise ValueError("runtime projection member slice must be non-empty")


@dataclass(frozen=True, slots=True)
class QuantizedLinearSpec:
    """Description of one frozen packed linear (src/nanoquant/runtime/backend.py:27-73)."""

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
    members: tuple[ProjectionMemberSpec, ...] = ()
    patch_rank: int = 0
    patch_value_dtype: str | None = None
    bias_dtype: str | None = None

    def __post_init__(self) -> None:
        problems = (
            (not _canonical_name(self.name), "runtime layer name must be a canonical dotted path"),
            (
                min(self.in_features, self.out_features, self.rank) <= 0,
                "runtime linear dimensions and rank must be positive",
            ),
            (
                not 0 <= self.outlier_count <= self.in_features,
                "runtime outlier count is outside the input dimension",
            ),
            (
                (self.outlier_count > 0) != (self.outlier_value_dtype is not None),
                "runtime outlier dtype must be present exactly when outliers are present",
            ),
            (
                self.has_outlier_scales and self.outlier_count == 0,
                "runtime outlier scales require outlier values",
            ),
            (
                not 0 <= self.patch_rank <= min(self.in_features, self.out_features),
                "runtime patch rank is outside the linear dimensions",
            ),
            (
                (self.patch_rank > 0) != (self.patch_value_dtype is not None),
                "runtime patch dtype must be present exactly when a patch is present",
            ),
            (
                self.bias_dtype is not None and not self.has_bias,
                "runtime bias dtype requires a bias",
            ),
        )
        for failed, message in problems:
            if failed:
                raise ValueError(message)
        if self.members:
            _check_members(self.members, self.out_features)


def _check_members(members: tuple[ProjectionMemberSpec, ...], out_features: int) -> None:
    names = [member.name for member in members]
    if len(members) < 2 or len(set(names)) != len(names):
        raise ValueError("runtime projection group members must be unique")
    expected_start = 0
    for member in members:
        if member.row_start != expected_start:
            raise ValueError("runtime projection group slices must be contiguous")
        expected_start = member.row_end
    if expected_start != out_features:
        raise ValueError("runtime projection group slices must cover the output")


@dataclass(frozen=True, slots=True)
class WorkloadSpec:
    """Execution geometry a plan is resolved for (src/nanoquant/runtime/backend.py:76-91)."""

    kind: WorkloadKind
    device_type: str
    input_dtype: str
    batch_size: int
    token_count: int
    deterministic: bool = False

    def __post_init__(self) -> None:
        if self.kind not in _WORKLOAD_KINDS:
            raise ValueError(f"unsupported runtime workload kind: {self.kind}")
        if not self.device_type:
            raise ValueError("runtime workload device type must be non-empty")
        if min(self.batch_size, self.token_count) <= 0:
            raise ValueError("runtime workload batch and token counts must be positive")


@dataclass(frozen=True, slots=True)
class BackendCapabilities:
    """Finite capability declaration (src/nanoquant/runtime/backend.py:94-121)."""

    logical_formats: tuple[str, ...]
    device_types: tuple[str, ...]
    input_dtypes: tuple[str, ...]
    factor_dtypes: tuple[str, ...]
    scale_dtypes: tuple[str, ...]
    outlier_value_dtypes: tuple[str, ...]
    workload_kinds: tuple[WorkloadKind, ...]
    supports_bias: bool
    supports_outliers: bool
    supports_deterministic: bool
    in_feature_alignment: int = 1
    out_feature_alignment: int = 1
    rank_alignment: int = 1
    maximum_batch_size: int | None = None
    maximum_token_count: int | None = None
    patch_value_dtypes: tuple[str, ...] = ()

    def __post_init__(self) -> None:
        if not (self.logical_formats and self.device_types and self.input_dtypes):
            raise ValueError(
                "runtime backend capabilities must declare formats, devices, and input dtypes"
            )
        alignments = (self.in_feature_alignment, self.out_feature_alignment, self.rank_alignment)
        if min(alignments) <= 0:
            raise ValueError("runtime backend alignments must be positive")
        if self.maximum_batch_size is not None and self.maximum_batch_size <= 0:
            raise ValueError("runtime backend maximum batch size must be positive")
        if self.maximum_token_count is not None and self.maximum_token_count <= 0:
            raise ValueError("runtime backend maximum token count must be positive")


@dataclass(frozen=True, slots=True)
class SupportResult:
    """Accept/reject answer with a stable code (src/nanoquant/runtime/backend.py:124-138)."""

    supported: bool
    code: str
    reason: str

    @classmethod
    def accepted(cls) -> SupportResult:
        return cls(True, "NQ-INF-OK", "supported")

    @classmethod
    def rejected(cls, code: str, reason: str) -> SupportResult:
        if not (code and reason):
            raise ValueError("runtime backend rejection requires a code and reason")
        return cls(False, code, reason)


@runtime_checkable
class RuntimeLayerState(Protocol):
    @property
    def spec(self) -> QuantizedLinearSpec: ...


@dataclass(frozen=True, slots=True)
class PreparedLayer:
    """Backend-owned device payload for one layer (src/nanoquant/runtime/backend.py:147-152)."""

    backend_name: str
    backend_version: str
    spec: QuantizedLinearSpec
    payload: object


@runtime_checkable
class RuntimeBackend(Protocol):
    """The protocol every backend implements (src/nanoquant/runtime/backend.py:155-166)."""

    name: str
    version: str

    def capabilities(self) -> BackendCapabilities: ...

    def supports(self, op: QuantizedLinearSpec, workload: WorkloadSpec) -> SupportResult: ...

    def prepare(self, state: RuntimeLayerState, device: DeviceLike) -> PreparedLayer: ...

    def linear(self, value: torch.Tensor, layer: PreparedLayer) -> torch.Tensor: ...


def _capability_checks(
    caps: BackendCapabilities, op: QuantizedLinearSpec, workload: WorkloadSpec
):
    """Yield ``(ok, code, reason)`` in the reference's order; the first failure wins."""

    yield (
        op.logical_format in caps.logical_formats,
        "NQ-INF-FORMAT",
        f"logical format {op.logical_format!r} is not supported",
    )
    yield (
        workload.device_type in caps.device_types,
        "NQ-INF-DEVICE",
        f"device type {workload.device_type!r} is not supported",
    )
    yield (
        workload.input_dtype in caps.input_dtypes,
        "NQ-INF-INPUT-DTYPE",
        f"input dtype {workload.input_dtype!r} is not supported",
    )
    yield (
        op.factor_dtype in caps.factor_dtypes,
        "NQ-INF-FACTOR-DTYPE",
        f"factor dtype {op.factor_dtype!r} is not supported",
    )
    yield (
        op.scale_dtype in caps.scale_dtypes,
        "NQ-INF-SCALE-DTYPE",
        f"scale dtype {op.scale_dtype!r} is not supported",
    )
    yield (
        workload.kind in caps.workload_kinds,
        "NQ-INF-WORKLOAD",
        f"workload kind {workload.kind!r} is not supported",
    )
    yield (not op.has_bias or caps.supports_bias, "NQ-INF-BIAS", "bias is not supported")
    yield (
        op.bias_dtype is None or op.bias_dtype in caps.scale_dtypes,
        "NQ-INF-BIAS-DTYPE",
        f"bias dtype {op.bias_dtype!r} is not supported",
    )
    yield (
        op.outlier_count == 0 or caps.supports_outliers,
        "NQ-INF-OUTLIERS",
        "salient outliers are not supported",
    )
    yield (
        op.outlier_value_dtype is None or op.outlier_value_dtype in caps.outlier_value_dtypes,
        "NQ-INF-OUTLIER-DTYPE",
        f"outlier dtype {op.outlier_value_dtype!r} is not supported",
    )
    yield (
        op.patch_value_dtype is None or op.patch_value_dtype in caps.patch_value_dtypes,
        "NQ-INF-PATCH",
        f"low-rank patch dtype {op.patch_value_dtype!r} is not supported",
    )
    yield (
        not workload.deterministic or caps.supports_deterministic,
        "NQ-INF-DETERMINISM",
        "deterministic execution is not supported",
    )
    for size, alignment, code, label in (
        (op.in_features, caps.in_feature_alignment, "NQ-INF-IN-ALIGNMENT", "input features"),
        (op.out_features, caps.out_feature_alignment, "NQ-INF-OUT-ALIGNMENT", "output features"),
        (op.rank, caps.rank_alignment, "NQ-INF-RANK-ALIGNMENT", "rank"),
    ):
        yield (size % alignment == 0, code, f"{label} must be aligned to {alignment}")
    yield (
        caps.maximum_batch_size is None or workload.batch_size <= caps.maximum_batch_size,
        "NQ-INF-BATCH",
        f"batch size {workload.batch_size} exceeds the backend maximum",
    )
    yield (
        caps.maximum_token_count is None or workload.token_count <= caps.maximum_token_count,
        "NQ-INF-TOKENS",
        f"token count {workload.token_count} exceeds the backend maximum",
    )


def evaluate_capabilities(
    capabilities: BackendCapabilities,
    op: QuantizedLinearSpec,
    workload: WorkloadSpec,
) -> SupportResult:
    """Return the first stable, actionable reason a backend cannot run ``op``
    (src/nanoquant/runtime/backend.py:169-266)."""

    for ok, code, reason in _capability_checks(capabilities, op, workload):
        if not ok:
            return SupportResult.rejected(code, reason)
    return SupportResult.accepted()
