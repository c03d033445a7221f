"""Packed sign-word layout ``llama.cpp-i32-lsb-v1`` and the packed layer state.

Layout (src/nanoquant/runtime/packed.py:84-218, Docs/19-nanoquant-packed-layout-v1.md:87-100):
a sign matrix ``[rows, cols]`` is stored as int32 words ``[rows, ceil(cols/32)]``;
column ``c`` lives in word ``c // 32`` at bit ``c % 32`` (least-significant bit
first); a set bit means -1, a clear bit +1, and the pad bits past ``cols`` are 0.

The host functions here are prepare-time utilities on CPU tensors (artifact
writing, ``to_logical``).  The device-side unpack is the HIP kernel behind
``nanoquant_amd.runtime.hip_backend.unpack_sign_matrix_device``.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from nanoquant_amd.runtime.backend import QuantizedLinearSpec
from nanoquant_amd.runtime.constants import PackedLayout
from nanoquant_amd.runtime.logical import (
    LogicalLayerState,
    canonical_torch_dtype,
    parse_torch_dtype,
)

PACKED_LAYOUT_VERSION = PackedLayout.LLAMA_CPP_I32_LSB_V1.value
PACKED_WORD_BITS = 32
PACKED_WORD_DTYPE = "int32"
PACKED_TENSOR_NAMESPACE = f"layouts.{PACKED_LAYOUT_VERSION}"

# Identity of the llama.cpp fork that defines the layout; these are format
# pins carried verbatim so artifacts written by either runtime declare the same
# provenance (src/nanoquant/runtime/packed.py:17-34).
PACKED_REFERENCE_REPOSITORY = "modified-llama.cpp"
PACKED_REFERENCE_COMMIT = "da52148384591f4b0d87d58c12862e30f43014f1"
PACKED_REFERENCE_DIRTY_DIFF_GIT_OBJECT = "cf463b9266db4e1f162ad8970e8ddcc1abfb5fbd"
PACKED_REFERENCE_CUDA_SHA256 = "5c87336c2b6b8fb33805c6ee6a8752d4bd364beed63fd4cca03c2b36be966619"
PACKED_REFERENCE_CONVERTER_SHA256 = (
    "c2e1fd064bbd46f38e9e3c5f739865d198ca75bd0bb9db16f72530d378d11304"
)
PACKED_REFERENCE_DOCUMENTATION_SHA256 = (
    "12c46863a480a04b1ba449bb7bcb2f637419b677678b60f93522c531bd3f9ac8"
)
PACKED_REFERENCE_MODEL_LOADER_SHA256 = (
    "11175fca67ecd8b97f6d6ffa7d2e8b848839d768669d63f7ec629a69d8d704aa"
)
PACKED_REFERENCE_CPU_SHA256 = "f51195610b4c533e4f606f984c7083bb542e4c3b3c8e740fdc647f8a5b0eff1c"

# GGUF sidecar tensor names per role (src/nanoquant/runtime/packed.py:35-45).
GGUF_TENSOR_SUFFIXES = (
    ("factor_right_words", "nq_v"),
    ("factor_left_words", "nq_u"),
    ("scale_pre", "nq_scale_pre"),
    ("scale_mid", "nq_scale_mid"),
    ("scale_post", "nq_scale_post"),
    ("outlier_indices", "nq_salient_idx"),
    ("outlier_values", "nq_salient_weight"),
    ("outlier_scales", "nq_salient_scale"),
    ("bias", "bias"),
)

_PROVENANCE_PINS = (
    PACKED_REFERENCE_REPOSITORY,
    PACKED_REFERENCE_COMMIT,
    PACKED_REFERENCE_DIRTY_DIFF_GIT_OBJECT,
    PACKED_REFERENCE_CUDA_SHA256,
    PACKED_REFERENCE_CONVERTER_SHA256,
    PACKED_REFERENCE_DOCUMENTATION_SHA256,
    PACKED_REFERENCE_MODEL_LOADER_SHA256,
    PACKED_REFERENCE_CPU_SHA256,
)


@dataclass(frozen=True, slots=True)
class PackedReferenceProvenance:
    """Schema-1 provenance of the layout (src/nanoquant/runtime/packed.py:48-81)."""

    repository: str = PACKED_REFERENCE_REPOSITORY
    commit: str = PACKED_REFERENCE_COMMIT
    dirty_diff_git_object: str = PACKED_REFERENCE_DIRTY_DIFF_GIT_OBJECT
    cuda_sha256: str = PACKED_REFERENCE_CUDA_SHA256
    converter_sha256: str = PACKED_REFERENCE_CONVERTER_SHA256
    documentation_sha256: str = PACKED_REFERENCE_DOCUMENTATION_SHA256
    model_loader_sha256: str = PACKED_REFERENCE_MODEL_LOADER_SHA256
    cpu_sha256: str = PACKED_REFERENCE_CPU_SHA256

    def __post_init__(self) -> None:
        declared = (
            self.repository,
            self.commit,
            self.dirty_diff_git_object,
            self.cuda_sha256,
            self.converter_sha256,
            self.documentation_sha256,
            self.model_loader_sha256,
            self.cpu_sha256,
        )
        if declared != _PROVENANCE_PINS:
            raise ValueError("packed layout reference provenance differs from schema 1")


@dataclass(frozen=True, slots=True)
class PackedLayoutMetadata:
    """The layout contract itself (src/nanoquant/runtime/packed.py:84-136)."""

    version: str = PACKED_LAYOUT_VERSION
    word_dtype: str = PACKED_WORD_DTYPE
    word_bits: int = PACKED_WORD_BITS
    bit_order: str = "least-significant-bit-first"
    positive_bit: int = 0
    negative_bit: int = 1
    padding_bit: int = 0
    minimum_alignment_bytes: int = 4
    vector_alignment_bytes: int = 16
    tensor_namespace: str = PACKED_TENSOR_NAMESPACE
    left_sidecar_name: str = "nq_u"
    right_sidecar_name: str = "nq_v"
    scale_pre_sidecar_name: str = "nq_scale_pre"
    scale_mid_sidecar_name: str = "nq_scale_mid"
    scale_post_sidecar_name: str = "nq_scale_post"
    outlier_index_sidecar_name: str = "nq_salient_idx"
    outlier_value_sidecar_name: str = "nq_salient_weight"
    outlier_scale_sidecar_name: str = "nq_salient_scale"
    bias_storage: str = "separate-additive-tensor"
    reference: PackedReferenceProvenance = PackedReferenceProvenance()

    def __post_init__(self) -> None:
        if self.version != PACKED_LAYOUT_VERSION:
            raise ValueError(f"unsupported packed layout version: {self.version}")
        if (self.word_dtype, self.word_bits) != (PACKED_WORD_DTYPE, PACKED_WORD_BITS):
            raise ValueError("packed layout word representation differs from the runtime")
        if self.bit_order != "least-significant-bit-first":
            raise ValueError("packed layout bit order differs from the runtime")
        if (self.positive_bit, self.negative_bit, self.padding_bit) != (0, 1, 0):
            raise ValueError("packed layout sign or padding encoding differs from the runtime")
        if (self.minimum_alignment_bytes, self.vector_alignment_bytes) != (4, 16):
            raise ValueError("packed layout alignment metadata differs from the reference kernel")
        if self.tensor_namespace != PACKED_TENSOR_NAMESPACE:
            raise ValueError("packed tensor namespace differs from the runtime")
        by_role = dict(GGUF_TENSOR_SUFFIXES)
        declared = {
            "factor_left_words": self.left_sidecar_name,
            "factor_right_words": self.right_sidecar_name,
            "scale_pre": self.scale_pre_sidecar_name,
            "scale_mid": self.scale_mid_sidecar_name,
            "scale_post": self.scale_post_sidecar_name,
            "outlier_indices": self.outlier_index_sidecar_name,
            "outlier_values": self.outlier_value_sidecar_name,
            "outlier_scales": self.outlier_scale_sidecar_name,
        }
        if any(by_role[role] != name for role, name in declared.items()):
            raise ValueError("packed GGUF sidecar names differ from the reference format")
        if self.bias_storage != "separate-additive-tensor":
            raise ValueError("packed bias storage differs from the runtime")
        if self.reference != PackedReferenceProvenance():
            raise ValueError("packed layout reference provenance differs from the runtime")


def packed_word_count(columns: int) -> int:
    """``ceil(columns / 32)`` (src/nanoquant/runtime/packed.py:139-142)."""

    if columns <= 0:
        raise ValueError("packed sign column count must be positive")
    return -(-columns // PACKED_WORD_BITS)


def packed_row_stride_bytes(columns: int) -> int:
    """Bytes per packed row (src/nanoquant/runtime/packed.py:145-146)."""

    return 4 * packed_word_count(columns)


def supports_vector_word_loads(words: torch.Tensor) -> bool:
    """The 16-byte vector-load predicate: 16-B aligned base and row stride
    (src/nanoquant/runtime/packed.py:149-158)."""

    if words.ndim != 2 or words.dtype != torch.int32 or not words.is_contiguous():
        return False
    row_bytes = words.stride(0) * words.element_size()
    return words.data_ptr() % 16 == 0 and row_bytes % 16 == 0


def _check_sign_matrix(signs: torch.Tensor) -> None:
    if signs.ndim != 2 or not signs.is_contiguous():
        raise ValueError("logical signs must be a contiguous matrix")
    if min(signs.shape) <= 0:
        raise ValueError("logical sign matrix dimensions must be positive")
    if not bool(((signs == 1) | (signs == -1)).all()):
        raise ValueError("logical signs contain a value other than -1 or +1")


def pack_sign_matrix(signs: torch.Tensor) -> torch.Tensor:
    """+/-1 ``[rows, cols]`` -> int32 words ``[rows, ceil(cols/32)]`` on the CPU
    (src/nanoquant/runtime/packed.py:170-186)."""

    _check_sign_matrix(signs)
    rows, columns = signs.shape
    words = packed_word_count(columns)
    negative = torch.zeros(rows, words * PACKED_WORD_BITS, dtype=torch.int64)
    negative[:, :columns] = (signs.detach().cpu() < 0).to(torch.int64)
    lanes = negative.view(rows, words, PACKED_WORD_BITS)
    accumulated = torch.zeros(rows, words, dtype=torch.int64)
    for bit in range(PACKED_WORD_BITS):
        accumulated |= lanes[:, :, bit] << bit
    wrapped = torch.where(accumulated >= 2**31, accumulated - 2**32, accumulated)
    return wrapped.to(torch.int32).contiguous()


def _check_packed_matrix(words: torch.Tensor, rows: int, columns: int) -> None:
    shape = (rows, packed_word_count(columns))
    if words.dtype != torch.int32 or tuple(words.shape) != shape or not words.is_contiguous():
        raise ValueError(
            f"packed sign matrix must be contiguous int32 with shape {shape}, got "
            f"{words.dtype} {tuple(words.shape)}"
        )
    tail = columns % PACKED_WORD_BITS
    if tail:
        pad_mask = (0xFFFFFFFF << tail) & 0xFFFFFFFF
        last = words[:, -1].to(torch.int64) & 0xFFFFFFFF
        if bool(((last & pad_mask) != 0).any()):
            raise ValueError("packed sign matrix has a non-zero padding bit")


def unpack_sign_matrix(
    words: torch.Tensor,
    rows: int,
    columns: int,
    *,
    dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """int32 words -> dense +/-1 ``[rows, columns]`` (src/nanoquant/runtime/packed.py:204-218).

    Host utility; device tensors go through the HIP unpack kernel
    (``hip_backend.unpack_sign_matrix_device``)."""

    _check_packed_matrix(words, rows, columns)
    unsigned = words.to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(PACKED_WORD_BITS, dtype=torch.int64, device=words.device)
    bits = (unsigned.unsqueeze(-1) >> shifts) & 1
    signs = 1 - 2 * bits.reshape(rows, -1)[:, :columns]
    return signs.to(dtype).contiguous()


def _factor_dtype(name: str) -> torch.dtype:
    if name not in ("float16", "bfloat16", "float32"):
        raise ValueError(f"packed layout does not support logical factor dtype: {name}")
    return parse_torch_dtype(name)


def _finite(tensor: torch.Tensor) -> bool:
    return bool(torch.isfinite(tensor).all())


@dataclass(frozen=True, slots=True)
class PackedLayerState:
    """Packed operand bundle and its invariants (src/nanoquant/runtime/packed.py:230-382).

    Salient ("outlier") columns index *input* features: ``outlier_indices[k] < in``,
    ``outlier_values`` is ``[out, k]`` and the stored ``scale_pre`` is exactly zero
    at those columns (src/nanoquant/runtime/packed.py:303-307).
    """

    spec: QuantizedLinearSpec
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

    def __post_init__(self) -> None:
        spec = self.spec
        if self.layout != PACKED_LAYOUT_VERSION:
            raise ValueError(f"unsupported packed layer layout: {self.layout}")
        _check_packed_matrix(self.left_words, spec.out_features, spec.rank)
        _check_packed_matrix(self.right_words, spec.rank, spec.in_features)
        for name, tensor, shape in (
            ("scale_pre", self.scale_pre, (spec.in_features,)),
            ("scale_mid", self.scale_mid, (spec.rank,)),
            ("scale_post", self.scale_post, (spec.out_features,)),
        ):
            if tuple(tensor.shape) != shape or not tensor.is_contiguous():
                raise ValueError(f"packed layer {name} shape or layout differs")
            if canonical_torch_dtype(tensor.dtype) != spec.scale_dtype:
                raise ValueError(f"packed layer {name} dtype differs")
            if not _finite(tensor):
                raise ValueError(f"packed layer {name} contains a non-finite value")
        self._check_bias()
        self._check_salient()
        self._check_patch()

    def _check_bias(self) -> None:
        spec = self.spec
        if (self.bias is not None) != spec.has_bias:
            raise ValueError("packed layer bias presence differs from its specification")
        if self.bias is None:
            return
        if tuple(self.bias.shape) != (spec.out_features,) or not self.bias.is_contiguous():
            raise ValueError("packed layer bias shape differs")
        if canonical_torch_dtype(self.bias.dtype) != (spec.bias_dtype or spec.scale_dtype):
            raise ValueError("packed layer bias dtype differs")
        if not _finite(self.bias):
            raise ValueError("packed layer bias contains a non-finite value")

    def _check_salient(self) -> None:
        spec = self.spec
        indices, values, scales = self.outlier_indices, self.outlier_values, self.outlier_scales
        if (indices is None) != (values is None):
            raise ValueError("packed layer outlier indices and values must be paired")
        if (indices is not None) != (spec.outlier_count > 0):
            raise ValueError("packed layer outlier presence differs from its specification")
        if indices is not None and values is not None:
            if indices.dtype != torch.int32:
                raise ValueError("packed llama.cpp salient indices must be int32")
            if tuple(indices.shape) != (spec.outlier_count,) or not indices.is_contiguous():
                raise ValueError("packed layer outlier index shape differs")
            value_shape = (spec.out_features, spec.outlier_count)
            if tuple(values.shape) != value_shape or not values.is_contiguous():
                raise ValueError("packed layer outlier value shape differs")
            if canonical_torch_dtype(values.dtype) != spec.outlier_value_dtype:
                raise ValueError("packed layer outlier value dtype differs")
            index = indices.to(torch.int64)
            if bool((index < 0).any()) or bool((index >= spec.in_features).any()):
                raise ValueError("packed layer outlier index is outside the input dimension")
            if not bool((index[1:] > index[:-1]).all()):
                raise ValueError("packed layer outlier indices must be strictly increasing")
            at_salient = self.scale_pre.index_select(0, index.to(self.scale_pre.device))
            if bool((at_salient != 0).any()):
                raise ValueError(
                    "packed llama.cpp salient columns require exactly zero scale_pre entries"
                )
            if values.dtype not in (torch.int8, torch.float16, torch.bfloat16, torch.float32):
                raise ValueError("packed llama.cpp salient value dtype is unsupported")
            if values.is_floating_point() and not _finite(values):
                raise ValueError("packed layer outlier value contains a non-finite value")
        if (scales is not None) != spec.has_outlier_scales:
            raise ValueError("packed layer outlier scale presence differs")
        if scales is not None:
            if values is None or values.dtype != torch.int8:
                raise ValueError("packed llama.cpp salient scales require int8 values")
            if tuple(scales.shape) != (spec.outlier_count,) or not scales.is_contiguous():
                raise ValueError("packed llama.cpp salient scales must have one value per column")
            if canonical_torch_dtype(scales.dtype) != spec.scale_dtype:
                raise ValueError("packed layer outlier scale dtype differs")
            if not _finite(scales):
                raise ValueError("packed layer outlier scale contains a non-finite value")
        if values is not None and values.dtype == torch.int8 and scales is None:
            raise ValueError("packed llama.cpp int8 salient values require scales")

    def _check_patch(self) -> None:
        spec = self.spec
        left, right = self.patch_left, self.patch_right
        if (left is None) != (right is None):
            raise ValueError("packed low-rank patch tensors must be paired")
        if (left is not None) != (spec.patch_rank > 0):
            raise ValueError("packed patch presence differs from its specification")
        if left is None or right is None:
            return
        if tuple(left.shape) != (spec.out_features, spec.patch_rank):
            raise ValueError("packed patch-left shape differs")
        if tuple(right.shape) != (spec.patch_rank, spec.in_features):
            raise ValueError("packed patch-right shape differs")
        if not (left.is_contiguous() and right.is_contiguous()):
            raise ValueError("packed low-rank patch tensors must be contiguous")
        if any(canonical_torch_dtype(t.dtype) != spec.patch_value_dtype for t in (left, right)):
            raise ValueError("packed patch dtype differs")
        if not (_finite(left) and _finite(right)):
            raise ValueError("packed low-rank patch contains a non-finite value")

    def to_logical(self) -> LogicalLayerState:
        """Unpack both factors into the logical state (src/nanoquant/runtime/packed.py:354-382)."""

        spec = self.spec
        factor = _factor_dtype(spec.factor_dtype)
        return LogicalLayerState(
            spec,
            unpack_sign_matrix(self.left_words, spec.out_features, spec.rank, dtype=factor),
            unpack_sign_matrix(self.right_words, spec.rank, spec.in_features, dtype=factor),
            self.scale_pre,
            self.scale_mid,
            self.scale_post,
            self.bias,
            self.outlier_indices,
            self.outlier_values,
            self.outlier_scales,
            self.patch_left,
            self.patch_right,
        )


def _host_copy(tensor: torch.Tensor | None) -> torch.Tensor | None:
    if tensor is None:
        return None
    return tensor.detach().cpu().clone().contiguous()


def pack_logical_layer(state: LogicalLayerState) -> PackedLayerState:
    """Logical +/-1 state -> packed state (src/nanoquant/runtime/packed.py:393-411)."""

    indices = _host_copy(state.outlier_indices)
    return PackedLayerState(
        state.spec,
        PACKED_LAYOUT_VERSION,
        pack_sign_matrix(state.left_binary),
        pack_sign_matrix(state.right_binary),
        _host_copy(state.scale_pre),
        _host_copy(state.scale_mid),
        _host_copy(state.scale_post),
        _host_copy(state.bias),
        None if indices is None else indices.to(torch.int32),
        _host_copy(state.outlier_values),
        _host_copy(state.outlier_scales),
        _host_copy(state.patch_left),
        _host_copy(state.patch_right),
    )
