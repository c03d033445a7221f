"""Compact right-factor codecs, expanded to canonical sign words at prepare time.

Two formats of the reference runtime are supported with their names, fields,
validation and host-side conversion (``to_packed``):

* mixed-V ``mixed-v-free-k10-pair9-v1`` (src/nanoquant/runtime/mixed_v.py:18-258):
  the first ``free_rows`` rows of V are canonical words; each other word is a
  19-bit record (10-bit index into a 1024-word codebook, 9-bit id of the pair
  of bits to flip, 496 valid pairs ``a < b``), records packed LSB-first;
* product codebook ``product-codebook-free-k16-v1``
  (src/nanoquant/runtime/product_codebook.py:27-283): each coded word is a
  16-bit index into the Cartesian product of two 256 x 16-bit sign tables; a
  factorization may be stored transposed (it is transposed back at prepare).

``HipPackedBackend.prepare`` expands both on the device
(``nq_decode_mixed_v_words``, ``nq_decode_product_codebook_words``,
``nq_transpose_signs``) instead of on the host; ``device_packed_state``
is that path.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from nanoquant_amd.runtime import _native
from nanoquant_amd.runtime.backend import QuantizedLinearSpec
from nanoquant_amd.runtime.packed import (
    PACKED_LAYOUT_VERSION,
    PACKED_WORD_BITS,
    PackedLayerState,
    pack_sign_matrix,
    packed_word_count,
    unpack_sign_matrix,
)

MIXED_V_FORMAT_VERSION = "mixed-v-free-k10-pair9-v1"
MIXED_V_INDEX_BITS = 10
MIXED_V_CORRECTION_BITS = 9
MIXED_V_RECORD_BITS = MIXED_V_INDEX_BITS + MIXED_V_CORRECTION_BITS
MIXED_V_CODEBOOK_SIZE = 1 << MIXED_V_INDEX_BITS
MIXED_V_CORRECTION_PAIR_COUNT = math.comb(PACKED_WORD_BITS, 2)

PRODUCT_CODEBOOK_FORMAT_VERSION = "product-codebook-free-k16-v1"
PRODUCT_CODEBOOK_INDEX_BITS = 16
PRODUCT_CODEBOOK_HALF_BITS = 16
PRODUCT_CODEBOOK_HALF_INDEX_BITS = 8
PRODUCT_CODEBOOK_TABLE_SIZE = 1 << PRODUCT_CODEBOOK_HALF_INDEX_BITS

_MASK32 = 0xFFFF_FFFF
_INT_DTYPES = (torch.int16, torch.int32, torch.int64)


# --- bit streams of fixed-width records -----------------------------------------
def _payload_words(count: int, bits: int) -> int:
    return (count * bits + PACKED_WORD_BITS - 1) // PACKED_WORD_BITS


def _pack_stream(records: torch.Tensor, bits: int) -> torch.Tensor:
    """Row-major unsigned records of `bits` bits, LSB-first, into int32 words."""

    values = records.reshape(-1).to(torch.int64)
    offsets = torch.arange(values.numel(), dtype=torch.int64) * bits
    word, shift = offsets // PACKED_WORD_BITS, offsets % PACKED_WORD_BITS
    out = torch.zeros(_payload_words(values.numel(), bits), dtype=torch.int64)
    out.index_add_(0, word, (values << shift) & _MASK32)
    spill = shift + bits > PACKED_WORD_BITS
    out.index_add_(0, word[spill] + 1, values[spill] >> (PACKED_WORD_BITS - shift[spill]))
    if bool((out > _MASK32).any()):
        raise AssertionError("record fields overlap")
    return out.to(torch.int32).contiguous()


def _unpack_stream(payload: torch.Tensor, count: int, bits: int) -> torch.Tensor:
    expected = _payload_words(count, bits)
    if payload.dtype != torch.int32 or tuple(payload.shape) != (expected,) or not payload.is_contiguous():
        raise ValueError(f"payload must be contiguous int32 with shape ({expected},)")
    words = payload.to(torch.int64) & _MASK32
    tail = (count * bits) % PACKED_WORD_BITS
    if tail and int(words[-1]) >> tail:
        raise ValueError("payload has a non-zero padding bit")
    offsets = torch.arange(count, dtype=torch.int64, device=payload.device) * bits
    word, shift = offsets // PACKED_WORD_BITS, offsets % PACKED_WORD_BITS
    values = words.index_select(0, word) >> shift
    spill = shift + bits > PACKED_WORD_BITS
    values[spill] |= words.index_select(0, word[spill] + 1) << (PACKED_WORD_BITS - shift[spill])
    return values & ((1 << bits) - 1)


# --- mixed-V ----------------------------------------------------------------------
def mixed_v_payload_word_count(record_count: int) -> int:
    if record_count <= 0:
        raise ValueError("mixed-V record count must be positive")
    return _payload_words(record_count, MIXED_V_RECORD_BITS)


def mixed_v_correction_pair_table(*, device: str | torch.device = "cpu") -> torch.Tensor:
    """Pair id -> ``a | b << 8`` for the lexicographic pairs ``a < b < 32`` (512
    entries; ids past 496 are zero)."""

    a, b = torch.triu_indices(PACKED_WORD_BITS, PACKED_WORD_BITS, offset=1)
    table = torch.zeros(1 << MIXED_V_CORRECTION_BITS, dtype=torch.int32)
    table[: a.numel()] = (a | (b << 8)).to(torch.int32)
    return table.to(device)


def _check_records(indices: torch.Tensor, pair_ids: torch.Tensor) -> None:
    if (indices.ndim != 2 or indices.shape != pair_ids.shape or indices.numel() == 0
            or not indices.is_contiguous() or not pair_ids.is_contiguous()):
        raise ValueError("mixed-V record fields must be matching non-empty contiguous matrices")
    if indices.dtype not in _INT_DTYPES or pair_ids.dtype not in _INT_DTYPES:
        raise ValueError("mixed-V record fields must use an integer dtype")
    if bool(((indices < 0) | (indices >= MIXED_V_CODEBOOK_SIZE)).any()):
        raise ValueError("mixed-V codebook index is outside the 10-bit codebook")
    if bool(((pair_ids < 0) | (pair_ids >= MIXED_V_CORRECTION_PAIR_COUNT)).any()):
        raise ValueError("mixed-V correction pair id is outside the 496 valid pairs")


def pack_mixed_v_records(codebook_indices: torch.Tensor, correction_pair_ids: torch.Tensor) -> torch.Tensor:
    _check_records(codebook_indices, correction_pair_ids)
    records = codebook_indices.cpu().to(torch.int64) | (correction_pair_ids.cpu().to(torch.int64) << MIXED_V_INDEX_BITS)
    return _pack_stream(records, MIXED_V_RECORD_BITS)


def unpack_mixed_v_records(payload: torch.Tensor, shape: tuple[int, int]) -> tuple[torch.Tensor, torch.Tensor]:
    if len(shape) != 2 or min(shape) <= 0:
        raise ValueError("mixed-V record shape must contain two positive dimensions")
    try:
        records = _unpack_stream(payload, shape[0] * shape[1], MIXED_V_RECORD_BITS)
    except ValueError as error:
        raise ValueError(f"mixed-V {error}") from None
    indices = (records & (MIXED_V_CODEBOOK_SIZE - 1)).reshape(shape).to(torch.int32).contiguous()
    pairs = (records >> MIXED_V_INDEX_BITS).reshape(shape).to(torch.int32).contiguous()
    _check_records(indices, pairs)
    return indices, pairs


def decode_mixed_v_right_words(free_right_words: torch.Tensor, coded_payload: torch.Tensor,
                               codebook_words: torch.Tensor, *, rank: int, in_features: int) -> torch.Tensor:
    """Host expansion to canonical right words ``[rank, wc(in)]``."""

    free_rows = int(free_right_words.shape[0])
    shape = (rank - free_rows, packed_word_count(in_features))
    indices, pair_ids = unpack_mixed_v_records(coded_payload, shape)
    pairs = mixed_v_correction_pair_table(device=coded_payload.device).index_select(0, pair_ids.reshape(-1).long())
    pairs = pairs.to(torch.int64)
    flips = (torch.ones_like(pairs) << (pairs & 0xFF)) | (torch.ones_like(pairs) << ((pairs >> 8) & 0xFF))
    base = codebook_words.index_select(0, indices.reshape(-1).long()).to(torch.int64) & _MASK32
    coded = (base ^ flips).to(torch.int32).reshape(shape)
    return torch.cat((free_right_words, coded), dim=0).contiguous()


@dataclass(frozen=True, slots=True)
class MixedVLayerState:
    spec: QuantizedLinearSpec
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

    def __post_init__(self) -> None:
        if self.format != MIXED_V_FORMAT_VERSION:
            raise ValueError(f"unsupported mixed-V format: {self.format}")
        if not 0 < self.free_rows < self.spec.rank:
            raise ValueError("mixed-V free row count must be between zero and rank")
        wpr = packed_word_count(self.spec.in_features)
        if tuple(self.free_right_words.shape) != (self.free_rows, wpr):
            raise ValueError("mixed-V free right-word shape differs")
        if self.free_right_words.dtype != torch.int32 or not self.free_right_words.is_contiguous():
            raise ValueError("mixed-V free right words must be contiguous int32")
        if tuple(self.codebook_words.shape) != (MIXED_V_CODEBOOK_SIZE,):
            raise ValueError("mixed-V codebook must contain exactly 1024 words")
        if self.codebook_words.dtype != torch.int32 or not self.codebook_words.is_contiguous():
            raise ValueError("mixed-V codebook words must be contiguous int32")
        self.to_packed()  # payload, pair ids, sign padding, scales and sidecars

    @property
    def coded_rows(self) -> int:
        return self.spec.rank - self.free_rows

    @property
    def record_count(self) -> int:
        return self.coded_rows * packed_word_count(self.spec.in_features)

    def to_packed(self) -> PackedLayerState:
        right = decode_mixed_v_right_words(self.free_right_words, self.coded_payload, self.codebook_words,
                                           rank=self.spec.rank, in_features=self.spec.in_features)
        return PackedLayerState(self.spec, PACKED_LAYOUT_VERSION, self.left_words, right, self.scale_pre,
                                self.scale_mid, self.scale_post, self.bias, self.outlier_indices,
                                self.outlier_values, self.outlier_scales, self.patch_left, self.patch_right)

    def to_logical(self):
        return self.to_packed().to_logical()


def mixed_v_from_packed_words(packed: PackedLayerState, *, free_rows: int, codebook_words: torch.Tensor,
                              codebook_indices: torch.Tensor, correction_pair_ids: torch.Tensor) -> MixedVLayerState:
    expected = (packed.spec.rank - free_rows, packed_word_count(packed.spec.in_features))
    if tuple(codebook_indices.shape) != expected or tuple(correction_pair_ids.shape) != expected:
        raise ValueError(f"mixed-V coded record matrices must have shape {expected}")
    state = MixedVLayerState(
        packed.spec, MIXED_V_FORMAT_VERSION, free_rows, packed.left_words,
        packed.right_words[:free_rows].contiguous(), pack_mixed_v_records(codebook_indices, correction_pair_ids),
        codebook_words.detach().cpu().to(torch.int32).contiguous(), packed.scale_pre, packed.scale_mid,
        packed.scale_post, packed.bias, packed.outlier_indices, packed.outlier_values, packed.outlier_scales,
        packed.patch_left, packed.patch_right,
    )
    if not torch.equal(state.to_packed().right_words, packed.right_words):
        raise ValueError("mixed-V records do not reconstruct the supplied packed right factor")
    return state


# --- product codebook -----------------------------------------------------------------
def product_codebook_payload_word_count(record_count: int) -> int:
    if record_count <= 0:
        raise ValueError("product-codebook record count must be positive")
    return _payload_words(record_count, PRODUCT_CODEBOOK_INDEX_BITS)


def pack_product_codebook_indices(indices: torch.Tensor) -> torch.Tensor:
    if indices.ndim != 2 or indices.numel() == 0 or not indices.is_contiguous() or indices.dtype not in _INT_DTYPES:
        raise ValueError("product-codebook indices must be a non-empty contiguous matrix")
    values = indices.cpu().to(torch.int64)
    if bool(((values < 0) | (values >= 1 << 16)).any()):
        raise ValueError("product-codebook index is outside the 16-bit range")
    return _pack_stream(values, PRODUCT_CODEBOOK_INDEX_BITS)


def unpack_product_codebook_indices(payload: torch.Tensor, shape: tuple[int, int]) -> torch.Tensor:
    if len(shape) != 2 or min(shape) <= 0:
        raise ValueError("product-codebook index shape must be positive")
    try:
        values = _unpack_stream(payload, shape[0] * shape[1], PRODUCT_CODEBOOK_INDEX_BITS)
    except ValueError as error:
        raise ValueError(f"product-codebook {error}".replace("padding bit", "padding record")) from None
    return values.reshape(shape).to(torch.int32).contiguous()


def pack_product_half_table(signs: torch.Tensor) -> torch.Tensor:
    """A 256 x 16 +-1 table as 256 int16 half-words (bit set = -1)."""

    if tuple(signs.shape) != (PRODUCT_CODEBOOK_TABLE_SIZE, PRODUCT_CODEBOOK_HALF_BITS) or not signs.is_contiguous():
        raise ValueError("product-codebook half table must have shape (256, 16)")
    if not bool(((signs == 1) | (signs == -1)).all()):
        raise ValueError("product-codebook half table contains a non-sign")
    bits = (signs.cpu() < 0).to(torch.int64) << torch.arange(PRODUCT_CODEBOOK_HALF_BITS)
    return bits.sum(dim=1).to(torch.int16).contiguous()


def unpack_product_half_table(words: torch.Tensor) -> torch.Tensor:
    if words.dtype != torch.int16 or tuple(words.shape) != (PRODUCT_CODEBOOK_TABLE_SIZE,) or not words.is_contiguous():
        raise ValueError("product-codebook half table must be contiguous int16[256]")
    bits = ((words.to(torch.int64) & 0xFFFF)[:, None] >> torch.arange(PRODUCT_CODEBOOK_HALF_BITS)) & 1
    return (1 - 2 * bits).to(torch.float32).contiguous()


def decode_product_codebook_right_words(free_right_words: torch.Tensor, coded_payload: torch.Tensor,
                                        first_half_words: torch.Tensor, second_half_words: torch.Tensor, *,
                                        rank: int, columns: int) -> torch.Tensor:
    free_rows = int(free_right_words.shape[0])
    wpr = packed_word_count(columns)
    if (not 0 < free_rows < rank or free_right_words.dtype != torch.int32
            or tuple(free_right_words.shape) != (free_rows, wpr) or not free_right_words.is_contiguous()):
        raise ValueError("product-codebook free right-word prefix is invalid")
    shape = (rank - free_rows, wpr)
    idx = unpack_product_codebook_indices(coded_payload, shape).to(torch.int64).reshape(-1)
    lo = first_half_words.to(torch.int64) & 0xFFFF
    hi = second_half_words.to(torch.int64) & 0xFFFF
    coded = (lo.index_select(0, idx & 0xFF) | (hi.index_select(0, idx >> 8) << 16)).to(torch.int32).reshape(shape)
    words = torch.cat((free_right_words, coded), dim=0).contiguous()
    unpack_sign_matrix(words, rank, columns)  # canonical zero tail padding
    return words


@dataclass(frozen=True, slots=True)
class ProductCodebookLayerState:
    spec: QuantizedLinearSpec
    format: str
    factorization_transposed: bool
    free_rows: int
    factor_left_words: torch.Tensor
    factor_right_free_words: torch.Tensor
    factor_right_coded_payload: torch.Tensor
    first_half_words: torch.Tensor
    second_half_words: torch.Tensor
    factor_scale_pre: torch.Tensor
    factor_scale_mid: torch.Tensor
    factor_scale_post: torch.Tensor
    outlier_indices: torch.Tensor | None = None
    outlier_values: torch.Tensor | None = None
    outlier_scales: torch.Tensor | None = None

    def __post_init__(self) -> None:
        spec = self.spec
        if self.format != PRODUCT_CODEBOOK_FORMAT_VERSION:
            raise ValueError(f"unsupported product-codebook format: {self.format}")
        if spec.has_bias or spec.patch_rank:
            raise ValueError("product-codebook v1 does not carry optional bias or patches")
        if not 0 < self.free_rows < spec.rank:
            raise ValueError("product-codebook free rows must be between zero and rank")
        left_shape = (self.factor_out_features, packed_word_count(spec.rank))
        if (self.factor_left_words.dtype != torch.int32 or tuple(self.factor_left_words.shape) != left_shape
                or not self.factor_left_words.is_contiguous()):
            raise ValueError("product-codebook factor-left words differ")
        unpack_sign_matrix(self.factor_left_words, self.factor_out_features, spec.rank)
        unpack_product_half_table(self.first_half_words)
        unpack_product_half_table(self.second_half_words)
        for name, value, size in (("factor_scale_pre", self.factor_scale_pre, self.factor_in_features),
                                  ("factor_scale_mid", self.factor_scale_mid, spec.rank),
                                  ("factor_scale_post", self.factor_scale_post, self.factor_out_features)):
            if (tuple(value.shape) != (size,) or not value.is_contiguous()
                    or str(value.dtype).removeprefix("torch.") != spec.scale_dtype
                    or not bool(torch.isfinite(value).all())):
                raise ValueError(f"product-codebook {name} differs")
        if (self.outlier_indices is None) != (self.outlier_values is None):
            raise ValueError("product-codebook outlier tensors must be paired")
        if (self.outlier_indices is None) != (spec.outlier_count == 0):
            raise ValueError("product-codebook outlier presence differs")
        self.to_packed()

    @property
    def factor_out_features(self) -> int:
        return self.spec.in_features if self.factorization_transposed else self.spec.out_features

    @property
    def factor_in_features(self) -> int:
        return self.spec.out_features if self.factorization_transposed else self.spec.in_features

    @property
    def coded_rows(self) -> int:
        return self.spec.rank - self.free_rows

    @property
    def record_count(self) -> int:
        return self.coded_rows * packed_word_count(self.factor_in_features)

    def to_packed(self) -> PackedLayerState:
        right = decode_product_codebook_right_words(
            self.factor_right_free_words, self.factor_right_coded_payload, self.first_half_words,
            self.second_half_words, rank=self.spec.rank, columns=self.factor_in_features)
        if self.factorization_transposed:
            f_left = unpack_sign_matrix(self.factor_left_words, self.factor_out_features, self.spec.rank)
            f_right = unpack_sign_matrix(right, self.spec.rank, self.factor_in_features)
            left_words = pack_sign_matrix(f_right.mT.contiguous())
            right_words = pack_sign_matrix(f_left.mT.contiguous())
            pre, post = self.factor_scale_post, self.factor_scale_pre
        else:
            left_words, right_words = self.factor_left_words, right
            pre, post = self.factor_scale_pre, self.factor_scale_post
        return PackedLayerState(self.spec, PACKED_LAYOUT_VERSION, left_words, right_words, pre, self.factor_scale_mid,
                                post, outlier_indices=self.outlier_indices, outlier_values=self.outlier_values,
                                outlier_scales=self.outlier_scales)

    def compact_logical_bits(self) -> int:
        spec = self.spec
        index_bits = math.ceil(math.log2(spec.in_features)) * spec.outlier_count
        value_bits = spec.out_features * spec.outlier_count * (8 if spec.outlier_value_dtype == "int8" else 16)
        scale_bits = spec.outlier_count * 16 if spec.has_outlier_scales else 0
        return (self.factor_left_words.numel() * 32 + self.factor_right_free_words.numel() * 32
                + self.record_count * PRODUCT_CODEBOOK_INDEX_BITS
                + 2 * PRODUCT_CODEBOOK_TABLE_SIZE * PRODUCT_CODEBOOK_HALF_BITS + 16
                + (self.factor_scale_pre.numel() + self.factor_scale_mid.numel() + self.factor_scale_post.numel()) * 16
                + index_bits + value_bits + scale_bits)


# --- device expansion (prepare) ----------------------------------------------------
def _dev(t: torch.Tensor | None, device: torch.device) -> torch.Tensor | None:
    return None if t is None else t.to(device).contiguous()


def _stream(device: torch.device) -> int:
    return _native.current_stream_handle(device)


def decode_mixed_v_on_device(state: MixedVLayerState, device: torch.device) -> torch.Tensor:
    spec = state.spec
    wpr = packed_word_count(spec.in_features)
    out = torch.empty((spec.rank, wpr), dtype=torch.int32, device=device)
    bad = torch.zeros(1, dtype=torch.int32, device=device)
    # Device copies stay referenced until the kernel is enqueued: a copy freed
    # earlier could be handed to the next copy before the kernel reads it.
    free, payload, book = (_dev(t, device) for t in (state.free_right_words, state.coded_payload,
                                                      state.codebook_words))
    status = _native.load().nq_decode_mixed_v_words(
        free.data_ptr(), state.free_rows, payload.data_ptr(), payload.numel(), book.data_ptr(), spec.rank,
        spec.in_features, out.data_ptr(), bad.data_ptr(), _stream(device))
    _native.check("nq_decode_mixed_v_words", status)
    if int(bad) != 0:
        raise ValueError("mixed-V correction pair id is outside the 496 valid pairs")
    return out


def transpose_signs_on_device(words: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    out = torch.empty((cols, packed_word_count(rows)), dtype=torch.int32, device=words.device)
    src = words.contiguous()
    status = _native.load().nq_transpose_signs(src.data_ptr(), rows, cols, out.data_ptr(), _stream(words.device))
    _native.check("nq_transpose_signs", status)
    return out


def decode_product_codebook_on_device(state: ProductCodebookLayerState,
                                      device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
    """(left_words, right_words) of the canonical orientation."""

    spec = state.spec
    columns = state.factor_in_features
    right = torch.empty((spec.rank, packed_word_count(columns)), dtype=torch.int32, device=device)
    free, payload, first, second = (_dev(t, device) for t in (
        state.factor_right_free_words, state.factor_right_coded_payload, state.first_half_words,
        state.second_half_words))
    status = _native.load().nq_decode_product_codebook_words(
        free.data_ptr(), state.free_rows, payload.data_ptr(), payload.numel(), first.data_ptr(), second.data_ptr(),
        spec.rank, columns, right.data_ptr(), _stream(device))
    _native.check("nq_decode_product_codebook_words", status)
    left = _dev(state.factor_left_words, device)
    if not state.factorization_transposed:
        return left, right
    return (transpose_signs_on_device(right, spec.rank, columns),
            transpose_signs_on_device(left, state.factor_out_features, spec.rank))


def device_packed_state(state: MixedVLayerState | ProductCodebookLayerState, device: torch.device) -> PackedLayerState:
    """The canonical ``PackedLayerState`` of a compact layer, expanded on `device`."""

    if isinstance(state, MixedVLayerState):
        return PackedLayerState(
            state.spec, PACKED_LAYOUT_VERSION, _dev(state.left_words, device), decode_mixed_v_on_device(state, device),
            _dev(state.scale_pre, device), _dev(state.scale_mid, device), _dev(state.scale_post, device),
            _dev(state.bias, device), _dev(state.outlier_indices, device), _dev(state.outlier_values, device),
            _dev(state.outlier_scales, device), _dev(state.patch_left, device), _dev(state.patch_right, device))
    left, right = decode_product_codebook_on_device(state, device)
    pre, post = ((state.factor_scale_post, state.factor_scale_pre) if state.factorization_transposed
                 else (state.factor_scale_pre, state.factor_scale_post))
    return PackedLayerState(
        state.spec, PACKED_LAYOUT_VERSION, left, right, _dev(pre, device), _dev(state.factor_scale_mid, device),
        _dev(post, device), outlier_indices=_dev(state.outlier_indices, device),
        outlier_values=_dev(state.outlier_values, device), outlier_scales=_dev(state.outlier_scales, device))
