"""Block-sharded packed model artifacts (the reference's on-disk format).

A packed artifact is a directory holding

* ``nanoquant-packed-model.json`` — the manifest: schema version, format name
  ``nanoquant-packed-model``, minimum runtime version, the layout contract
  (``PackedLayoutMetadata``), model metadata, the SHA-256 of the logical
  descriptor it was converted from, and per block its shard path, byte size,
  SHA-256 and layers (``QuantizedLinearSpec`` plus one entry per tensor role);
* ``weights/block-NNNNN.safetensors`` — one shard per block, tensors keyed
  ``layouts.llama.cpp-i32-lsb-v1.<layer>.<role>``.

The format, field names and validation rules follow
src/nanoquant/runtime/packed_artifact.py:40-223,285-344 and
src/nanoquant/runtime/artifact.py:23-66,200-226,488-494, so artifacts written
by the reference open here and vice versa. ``open_packed_artifact`` checks the
manifest, every shard's size and hash and every tensor header without loading
payloads; ``OpenPackedArtifact.load_layer`` reads one layer's tensors (to any
device) as a ``PackedLayerState`` for ``HipPackedBackend.prepare``.
"""

from __future__ import annotations

import hashlib
import json
import os
import shutil
import tempfile
import types
from collections.abc import Iterable, Mapping, Sequence
from dataclasses import MISSING, asdict, dataclass, fields, is_dataclass
from pathlib import Path, PurePosixPath
from typing import Any, get_args, get_origin, get_type_hints

import torch
from safetensors import safe_open
from safetensors.torch import save_file

from nanoquant_amd.runtime.backend import ProjectionMemberSpec, QuantizedLinearSpec  # noqa: F401 (decoder types)
from nanoquant_amd.runtime.constants import RUNTIME_ARTIFACT_SCHEMA_VERSION
from nanoquant_amd.runtime.logical import canonical_torch_dtype
from nanoquant_amd.runtime.packed import (
    PACKED_TENSOR_NAMESPACE,
    PackedLayerState,
    PackedLayoutMetadata,
    PackedReferenceProvenance,  # noqa: F401 (decoder types)
    packed_word_count,
)

PACKED_DESCRIPTOR_NAME = "nanoquant-packed-model.json"
PACKED_ARTIFACT_FORMAT = "nanoquant-packed-model"
MINIMUM_RUNTIME_VERSION = "0.1.0"
_DESCRIPTOR_LIMIT = 16 * 1024 * 1024
TENSOR_ROLES = (
    "factor_left_words",
    "factor_right_words",
    "scale_pre",
    "scale_mid",
    "scale_post",
    "bias",
    "outlier_indices",
    "outlier_values",
    "outlier_scales",
    "patch_left",
    "patch_right",
)
_SAFETENSORS_DTYPES = {
    "F16": "float16", "BF16": "bfloat16", "F32": "float32", "F64": "float64",
    "I8": "int8", "I16": "int16", "I32": "int32", "I64": "int64", "U8": "uint8", "BOOL": "bool",
}


class PackedArtifactError(ValueError):
    """A packed artifact that is missing, corrupt or inconsistent with its manifest."""


def _is_sha256(value: str) -> bool:
    return len(value) == 64 and all(ch in "0123456789abcdef" for ch in value)


def _check_relative(value: str) -> None:
    path = PurePosixPath(value)
    canonical = (
        bool(value) and "\\" not in value and not path.is_absolute()
        and all(part not in ("", ".", "..") for part in path.parts) and path.as_posix() == value
    )
    if not canonical:
        raise ValueError(f"artifact path is not canonical and relative: {value!r}")


@dataclass(frozen=True, slots=True)
class RuntimeModelMetadata:
    source: str
    revision: str
    family: str
    config_hash: str
    tokenizer_hash: str

    def __post_init__(self) -> None:
        if not all((self.source, self.revision, self.family, self.config_hash, self.tokenizer_hash)):
            raise ValueError("runtime model metadata fields must be non-empty")


@dataclass(frozen=True, slots=True)
class PackedTensorEntry:
    role: str
    key: str
    shape: tuple[int, ...]
    dtype: str

    def __post_init__(self) -> None:
        if self.role not in TENSOR_ROLES:
            raise ValueError(f"unsupported packed tensor role: {self.role}")
        if not self.key or self.key.startswith("/"):
            raise ValueError("packed tensor key must be non-empty and relative")
        if any(d < 0 for d in self.shape):
            raise ValueError("packed tensor dimensions must be non-negative")
        if not self.dtype:
            raise ValueError("packed tensor dtype must be non-empty")


def expected_tensors(spec: QuantizedLinearSpec) -> dict[str, tuple[tuple[int, ...], str]]:
    """Role -> (shape, dtype) a packed layer of `spec` must store."""

    out = {
        "factor_left_words": ((spec.out_features, packed_word_count(spec.rank)), "int32"),
        "factor_right_words": ((spec.rank, packed_word_count(spec.in_features)), "int32"),
        "scale_pre": ((spec.in_features,), spec.scale_dtype),
        "scale_mid": ((spec.rank,), spec.scale_dtype),
        "scale_post": ((spec.out_features,), spec.scale_dtype),
    }
    if spec.has_bias:
        out["bias"] = ((spec.out_features,), spec.bias_dtype or spec.scale_dtype)
    if spec.outlier_count:
        out["outlier_indices"] = ((spec.outlier_count,), "int32")
        out["outlier_values"] = ((spec.out_features, spec.outlier_count), str(spec.outlier_value_dtype))
    if spec.has_outlier_scales:
        out["outlier_scales"] = ((spec.outlier_count,), spec.scale_dtype)
    if spec.patch_rank:
        out["patch_left"] = ((spec.out_features, spec.patch_rank), str(spec.patch_value_dtype))
        out["patch_right"] = ((spec.patch_rank, spec.in_features), str(spec.patch_value_dtype))
    return out


@dataclass(frozen=True, slots=True)
class PackedLayerEntry:
    spec: QuantizedLinearSpec
    tensors: tuple[PackedTensorEntry, ...]

    def __post_init__(self) -> None:
        by_role = {t.role: t for t in self.tensors}
        if len(by_role) != len(self.tensors):
            raise ValueError(f"packed layer tensor roles are duplicated: {self.spec.name}")
        expected = expected_tensors(self.spec)
        if set(by_role) != set(expected):
            raise ValueError(f"packed layer tensor inventory differs from its specification: {self.spec.name}")
        for role, (shape, dtype) in expected.items():
            entry = by_role[role]
            if entry.key != f"{PACKED_TENSOR_NAMESPACE}.{self.spec.name}.{role}":
                raise ValueError(f"packed layer tensor key differs: {self.spec.name}:{role}")
            if entry.shape != shape or entry.dtype != dtype:
                raise ValueError(f"packed layer tensor metadata differs: {self.spec.name}:{role}")


@dataclass(frozen=True, slots=True)
class PackedBlockEntry:
    index: int
    path: str
    bytes: int
    sha256: str
    layers: tuple[PackedLayerEntry, ...]

    def __post_init__(self) -> None:
        if self.index < 0:
            raise ValueError("packed block index must be non-negative")
        if self.bytes <= 0:
            raise ValueError("packed block shard must be non-empty")
        if not _is_sha256(self.sha256):
            raise ValueError("packed block hash must be a lowercase SHA-256 digest")
        _check_relative(self.path)
        names = [layer.spec.name for layer in self.layers]
        if not names or len(names) != len(set(names)):
            raise ValueError("packed block must contain uniquely named layers")


@dataclass(frozen=True, slots=True)
class PackedModelManifest:
    schema_version: int
    artifact_format: str
    minimum_runtime_version: str
    layout: PackedLayoutMetadata
    model: RuntimeModelMetadata
    logical_descriptor_sha256: str
    blocks: tuple[PackedBlockEntry, ...]
    layer_count: int
    weight_bytes: int

    def __post_init__(self) -> None:
        if self.schema_version != RUNTIME_ARTIFACT_SCHEMA_VERSION:
            raise ValueError(f"unsupported packed artifact schema: {self.schema_version}")
        if self.artifact_format != PACKED_ARTIFACT_FORMAT:
            raise ValueError(f"unsupported packed artifact format: {self.artifact_format}")
        if self.minimum_runtime_version != MINIMUM_RUNTIME_VERSION:
            raise ValueError(f"unsupported packed minimum runtime version: {self.minimum_runtime_version}")
        if not _is_sha256(self.logical_descriptor_sha256):
            raise ValueError("packed source descriptor hash must be lowercase SHA-256")
        indexes = [b.index for b in self.blocks]
        if not indexes or indexes != list(range(len(indexes))):
            raise ValueError(f"packed artifact blocks are not contiguous: {indexes}")
        names = [layer.spec.name for b in self.blocks for layer in b.layers]
        if len(names) != len(set(names)) or len(names) != self.layer_count:
            raise ValueError("packed artifact layer count or uniqueness is inconsistent")
        if sum(b.bytes for b in self.blocks) != self.weight_bytes:
            raise ValueError("packed artifact weight byte count is inconsistent")


# --- strict JSON -> dataclass decoding ------------------------------------------
def _from_json(value: object, annotation: Any, path: str) -> object:
    origin, args = get_origin(annotation), get_args(annotation)
    if origin is types.UnionType:
        if value is None and type(None) in args:
            return None
        last: ValueError | None = None
        for option in (a for a in args if a is not type(None)):
            try:
                return _from_json(value, option, path)
            except ValueError as error:
                last = error
        raise ValueError(f"{path}: value matches no allowed type") from last
    if origin is tuple:
        if not isinstance(value, list):
            raise ValueError(f"{path}: expected an array")
        if len(args) == 2 and args[1] is Ellipsis:
            return tuple(_from_json(item, args[0], f"{path}[{i}]") for i, item in enumerate(value))
        if len(value) != len(args):
            raise ValueError(f"{path}: expected {len(args)} items")
        return tuple(_from_json(item, a, f"{path}[{i}]") for i, (item, a) in enumerate(zip(value, args)))
    if isinstance(annotation, type) and is_dataclass(annotation):
        if not isinstance(value, dict):
            raise ValueError(f"{path}: expected an object")
        known = {f.name: f for f in fields(annotation)}
        unknown = sorted(set(value) - set(known))
        if unknown:
            raise ValueError(f"{path}: unknown fields {unknown}")
        hints = get_type_hints(annotation)
        kwargs = {}
        for name, f in known.items():
            if name in value:
                kwargs[name] = _from_json(value[name], hints[name], f"{path}.{name}")
            elif f.default is MISSING and f.default_factory is MISSING:
                raise ValueError(f"{path}.{name}: required field is missing")
        return annotation(**kwargs)
    for scalar in (bool, int, str):
        if annotation is scalar:
            if not isinstance(value, scalar) or (scalar is int and isinstance(value, bool)):
                raise ValueError(f"{path}: expected {scalar.__name__}")
            return value
    if annotation is float:
        if isinstance(value, bool) or not isinstance(value, (int, float)):
            raise ValueError(f"{path}: expected a number")
        return float(value)
    raise ValueError(f"{path}: unsupported annotation {annotation!r}")


def decode_manifest(payload: object) -> PackedModelManifest:
    return _from_json(payload, PackedModelManifest, "manifest")  # type: ignore[return-value]


def _sha256_file(path: Path) -> str:
    digest = hashlib.sha256()
    with path.open("rb") as stream:
        for chunk in iter(lambda: stream.read(1 << 20), b""):
            digest.update(chunk)
    return digest.hexdigest()


def _member(root: Path, relative: str) -> Path:
    _check_relative(relative)
    candidate = (root / relative).resolve()
    if root.resolve() not in candidate.parents:
        raise PackedArtifactError(f"packed artifact member escapes its root: {relative}")
    return candidate


# --- reading --------------------------------------------------------------------
@dataclass(frozen=True, slots=True)
class OpenPackedArtifact:
    root: Path
    manifest: PackedModelManifest

    def layer_names(self) -> list[str]:
        return [layer.spec.name for block in self.manifest.blocks for layer in block.layers]

    def load_layer(self, name: str, device: torch.device | str = "cpu") -> PackedLayerState:
        """One layer's tensors from its shard as a ``PackedLayerState`` on `device`
        (src/nanoquant/runtime/packed_artifact.py:191-223)."""

        hits = [(b, layer) for b in self.manifest.blocks for layer in b.layers if layer.spec.name == name]
        if len(hits) != 1:
            raise KeyError(f"packed artifact layer not found: {name}")
        block, layer = hits[0]
        tensors: dict[str, torch.Tensor] = {}
        with safe_open(str(self.root / block.path), framework="pt", device="cpu") as handle:
            available = set(handle.keys())
            for entry in layer.tensors:
                if entry.key not in available:
                    raise PackedArtifactError(f"packed artifact tensor is missing: {entry.key}")
                value = handle.get_tensor(entry.key)
                tensors[entry.role] = value.to(device) if torch.device(device).type != "cpu" else value
        return PackedLayerState(
            layer.spec, self.manifest.layout.version, tensors["factor_left_words"], tensors["factor_right_words"],
            tensors["scale_pre"], tensors["scale_mid"], tensors["scale_post"], tensors.get("bias"),
            tensors.get("outlier_indices"), tensors.get("outlier_values"), tensors.get("outlier_scales"),
            tensors.get("patch_left"), tensors.get("patch_right"),
        )


def open_packed_artifact(root: str | Path, *, verify_hashes: bool = True) -> OpenPackedArtifact:
    """Validate the manifest, every shard's presence, size and (optionally) hash,
    and every tensor header, without loading tensor payloads
    (src/nanoquant/runtime/packed_artifact.py:299-344)."""

    base = Path(root)
    descriptor = base / PACKED_DESCRIPTOR_NAME
    if not descriptor.is_file():
        raise PackedArtifactError("packed artifact descriptor is missing")
    if descriptor.stat().st_size > _DESCRIPTOR_LIMIT:
        raise PackedArtifactError("packed artifact descriptor exceeds the size limit")
    try:
        manifest = decode_manifest(json.loads(descriptor.read_text(encoding="utf-8")))
    except (OSError, UnicodeError, json.JSONDecodeError, KeyError, TypeError, ValueError) as error:
        raise PackedArtifactError(f"packed artifact descriptor is invalid: {error}") from error
    for block in manifest.blocks:
        shard = _member(base, block.path)
        if not shard.is_file() or shard.stat().st_size != block.bytes:
            raise PackedArtifactError(f"packed artifact shard size or presence differs: {block.path}")
        if verify_hashes and _sha256_file(shard) != block.sha256:
            raise PackedArtifactError(f"packed artifact shard hash differs: {block.path}")
        declared = {t.key: t for layer in block.layers for t in layer.tensors}
        if len(declared) != sum(len(layer.tensors) for layer in block.layers):
            raise PackedArtifactError(f"packed artifact tensor key is duplicated: {block.path}")
        try:
            with safe_open(str(shard), framework="pt", device="cpu") as handle:
                if set(handle.keys()) != set(declared):
                    raise PackedArtifactError(f"packed artifact shard tensor inventory differs: {block.path}")
                for key, entry in declared.items():
                    view = handle.get_slice(key)
                    dtype = _SAFETENSORS_DTYPES.get(str(view.get_dtype()))
                    if tuple(view.get_shape()) != entry.shape or dtype != entry.dtype:
                        raise PackedArtifactError(f"packed artifact tensor header differs: {block.path}:{key}")
        except PackedArtifactError:
            raise
        except Exception as error:  # safetensors raises its own error types
            raise PackedArtifactError(f"packed artifact shard header is invalid: {block.path}") from error
    return OpenPackedArtifact(base.resolve(), manifest)


# --- writing --------------------------------------------------------------------
def _layer_tensors(state: PackedLayerState) -> list[tuple[str, torch.Tensor]]:
    roles = (
        ("factor_left_words", state.left_words), ("factor_right_words", state.right_words),
        ("scale_pre", state.scale_pre), ("scale_mid", state.scale_mid), ("scale_post", state.scale_post),
        ("bias", state.bias), ("outlier_indices", state.outlier_indices), ("outlier_values", state.outlier_values),
        ("outlier_scales", state.outlier_scales), ("patch_left", state.patch_left), ("patch_right", state.patch_right),
    )
    return [(role, value) for role, value in roles if value is not None]


def write_packed_artifact(
    output: str | Path,
    model: RuntimeModelMetadata,
    logical_descriptor_sha256: str,
    blocks: Mapping[int, Sequence[PackedLayerState]] | Iterable[tuple[int, Sequence[PackedLayerState]]],
) -> OpenPackedArtifact:
    """Write blocks 0..n-1 as shards plus the manifest, atomically (the directory
    appears only when complete); refuses to overwrite
    (src/nanoquant/runtime/packed_artifact.py:243-297)."""

    destination = Path(output)
    if destination.exists():
        raise FileExistsError(f"packed artifact output already exists: {destination}")
    items = sorted(blocks.items()) if isinstance(blocks, Mapping) else list(blocks)
    destination.parent.mkdir(parents=True, exist_ok=True)
    staging = Path(tempfile.mkdtemp(prefix=".nanoquant-packed-", dir=destination.parent))
    try:
        (staging / "weights").mkdir()
        entries, seen = [], set()
        for expected, (index, states) in enumerate(items):
            if index != expected:
                raise ValueError(f"packed artifact blocks must be contiguous: expected {expected}, received {index}")
            if not states:
                raise ValueError(f"packed artifact block {index} contains no layers")
            shard_tensors: dict[str, torch.Tensor] = {}
            layer_entries = []
            for state in states:
                if state.spec.name in seen:
                    raise ValueError(f"packed artifact layer name is duplicated: {state.spec.name}")
                seen.add(state.spec.name)
                tensor_entries = []
                for role, value in _layer_tensors(state):
                    key = f"{PACKED_TENSOR_NAMESPACE}.{state.spec.name}.{role}"
                    host = value.detach().cpu().contiguous()
                    shard_tensors[key] = host
                    tensor_entries.append(PackedTensorEntry(role, key, tuple(host.shape), canonical_torch_dtype(host.dtype)))
                layer_entries.append(PackedLayerEntry(state.spec, tuple(tensor_entries)))
            relative = f"weights/block-{index:05d}.safetensors"
            save_file(shard_tensors, str(staging / relative))
            shard = staging / relative
            entries.append(PackedBlockEntry(index, relative, shard.stat().st_size, _sha256_file(shard),
                                            tuple(layer_entries)))
        if not entries:
            raise ValueError("packed artifact must contain at least one block")
        manifest = PackedModelManifest(
            RUNTIME_ARTIFACT_SCHEMA_VERSION, PACKED_ARTIFACT_FORMAT, MINIMUM_RUNTIME_VERSION,
            PackedLayoutMetadata(), model, logical_descriptor_sha256, tuple(entries), len(seen),
            sum(e.bytes for e in entries),
        )
        with (staging / PACKED_DESCRIPTOR_NAME).open("w", encoding="utf-8", newline="\n") as stream:
            json.dump(asdict(manifest), stream, sort_keys=True, indent=2)
            stream.write("\n")
            stream.flush()
            os.fsync(stream.fileno())
        os.replace(staging, destination)
    except BaseException:
        shutil.rmtree(staging, ignore_errors=True)
        raise
    return open_packed_artifact(destination)
