"""CPU oracle for the packed binary low-rank linear — TEST INFRASTRUCTURE ONLY.

This module checks the product and is never part of it: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it. The shipped path (``nanoquant_amd``) never imports it and has no CPU
fallback.

It restates the reference algorithm:

* sign-word packing and unpacking of layout ``llama.cpp-i32-lsb-v1`` in numpy
  (src/nanoquant/runtime/packed.py:170-218): column ``c`` is bit ``c % 32`` of
  word ``c // 32``, set bit = -1, pad bits 0;
* the torch runtime forward ``PackedReferenceBackend.linear`` evaluated on
  ``x.float()`` (src/nanoquant/runtime/reference.py:93-106,184-235): unpack once,
  ``latent = F.linear(x * pre_masked, V)``,
  ``y = F.linear(latent * s_mid, U * s_out[:, None])``, plus salient columns,
  patch and bias — the "reference fp32 torch forward" parity is measured
  against;
* the dense reconstruction ``DenseReferenceBackend.linear``
  (src/nanoquant/runtime/reference.py:122-138), used to cross-check the above.

Pinning (what fixes each function independently of this code):
  pack_signs / unpack_signs — known-answer words and round-trip/padding cases of
    tests/unit/test_runtime_packed.py:27-68, the C restatement in
    ``nq_oracle.c`` (bit-exact cross-check) and exact integer arithmetic.
  packed_forward — exact rational evaluation (Fraction) of the reference test
    fixtures committed in tests/golden/, the dense reconstruction, and closed
    forms (all-+1 factors, one-hot rows, linearity, single-bit flips).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch
from torch.nn import functional as F

WORD_BITS = 32


def word_count(columns: int) -> int:
    """``ceil(columns / 32)`` (src/nanoquant/runtime/packed.py:139-142)."""

    if columns <= 0:
        raise ValueError("column count must be positive")
    return (columns + WORD_BITS - 1) // WORD_BITS


def pack_signs(signs: np.ndarray) -> np.ndarray:
    """+/-1 ``[rows, cols]`` -> int32 words (src/nanoquant/runtime/packed.py:170-186)."""

    signs = np.asarray(signs)
    if signs.ndim != 2 or not np.all((signs == 1) | (signs == -1)):
        raise ValueError("signs must be a +/-1 matrix")
    rows, cols = signs.shape
    words = word_count(cols)
    negative = np.zeros((rows, words * WORD_BITS), dtype=np.uint64)
    negative[:, :cols] = signs < 0
    weights = np.left_shift(np.uint64(1), np.arange(WORD_BITS, dtype=np.uint64))
    packed = (negative.reshape(rows, words, WORD_BITS) * weights).sum(axis=-1, dtype=np.uint64)
    return packed.astype(np.uint32).view(np.int32)


def padding_ok(words: np.ndarray, cols: int) -> bool:
    """Pad bits past ``cols`` must be zero (src/nanoquant/runtime/packed.py:196-201)."""

    tail = cols % WORD_BITS
    if tail == 0:
        return True
    last = np.asarray(words).view(np.uint32)[:, -1]
    return bool(np.all((last >> np.uint32(tail)) == 0))


def unpack_signs(words: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """int32 words -> int8 +/-1 ``[rows, cols]`` (src/nanoquant/runtime/packed.py:204-218)."""

    words = np.ascontiguousarray(words)
    if words.dtype != np.int32 or words.shape != (rows, word_count(cols)):
        raise ValueError("packed words must be int32 [rows, ceil(cols/32)]")
    if not padding_ok(words, cols):
        raise ValueError("packed sign matrix has a non-zero padding bit")
    unsigned = words.view(np.uint32)
    bits = (unsigned[:, :, None] >> np.arange(WORD_BITS, dtype=np.uint32)) & np.uint32(1)
    flat = bits.reshape(rows, -1)[:, :cols].astype(np.int8)
    return (1 - 2 * flat).astype(np.int8)


@dataclass
class PackedOperands:
    """One packed layer on the host, in the reference's tensor roles."""

    in_features: int
    out_features: int
    rank: int
    left_words: np.ndarray  # U [out, wc(rank)]
    right_words: np.ndarray  # V [rank, wc(in)]
    scale_pre: torch.Tensor
    scale_mid: torch.Tensor
    scale_post: torch.Tensor
    bias: torch.Tensor | None = None
    outlier_indices: torch.Tensor | None = None
    outlier_values: torch.Tensor | None = None
    outlier_scales: torch.Tensor | None = None
    patch_left: torch.Tensor | None = None
    patch_right: torch.Tensor | None = None


def _masked_pre(op: PackedOperands) -> torch.Tensor:
    """``scale_pre`` with salient columns zeroed (src/nanoquant/runtime/reference.py:101-106)."""

    pre = op.scale_pre.float().clone()
    if op.outlier_indices is not None and op.outlier_indices.numel():
        pre[op.outlier_indices.long()] = 0.0
    return pre


def _salient_weights(op: PackedOperands) -> torch.Tensor | None:
    """``outlier_values * outlier_scales`` (src/nanoquant/runtime/reference.py:93-98)."""

    if op.outlier_values is None:
        return None
    weights = op.outlier_values.float()
    if op.outlier_scales is not None:
        weights = weights * op.outlier_scales.float()
    return weights


class CpuPackedForward:
    """``PackedReferenceBackend`` restated: unpack once at construction, then each
    call is two fp32 ``F.linear`` over dense +/-1 factors plus the sidecars
    (src/nanoquant/runtime/reference.py:196-235). Also the CPU baseline."""

    def __init__(self, op: PackedOperands, *, compute_dtype: torch.dtype = torch.float32) -> None:
        self.op = op
        self.dtype = compute_dtype
        u = unpack_signs(op.left_words, op.out_features, op.rank)
        v = unpack_signs(op.right_words, op.rank, op.in_features)
        self.left = torch.from_numpy(u).to(compute_dtype)
        self.right = torch.from_numpy(v).to(compute_dtype)
        self.left_scaled = self.left * op.scale_post.to(compute_dtype).reshape(-1, 1)
        self.pre = _masked_pre(op).to(compute_dtype)
        self.mid = op.scale_mid.to(compute_dtype)
        sal = _salient_weights(op)
        self.salient = None if sal is None else sal.to(compute_dtype)
        self.patch_left = None if op.patch_left is None else op.patch_left.to(compute_dtype)
        self.patch_right = None if op.patch_right is None else op.patch_right.to(compute_dtype)
        self.bias = None if op.bias is None else op.bias.to(compute_dtype)

    def __call__(self, value: torch.Tensor) -> torch.Tensor:
        x = value.to(self.dtype)
        latent = F.linear(x * self.pre, self.right)
        out = F.linear(latent * self.mid, self.left_scaled)
        if self.salient is not None and self.op.outlier_indices is not None:
            out = out + F.linear(x.index_select(-1, self.op.outlier_indices.long()), self.salient)
        if self.patch_left is not None and self.patch_right is not None:
            out = out + F.linear(F.linear(x, self.patch_right), self.patch_left)
        if self.bias is not None:
            out = out + self.bias
        return out


def packed_forward(op: PackedOperands, value: torch.Tensor, *, dtype=torch.float32) -> torch.Tensor:
    """One-shot form of ``CpuPackedForward`` (``dtype=torch.float64`` for a tighter check)."""

    return CpuPackedForward(op, compute_dtype=dtype)(value)


def dense_forward(op: PackedOperands, value: torch.Tensor, *, dtype=torch.float64) -> torch.Tensor:
    """Dense reconstruction ``W = (U*s_out)(V*s_mid*pre)`` + salient columns + patch
    (src/nanoquant/runtime/reference.py:122-138)."""

    u = torch.from_numpy(unpack_signs(op.left_words, op.out_features, op.rank)).to(dtype)
    v = torch.from_numpy(unpack_signs(op.right_words, op.rank, op.in_features)).to(dtype)
    pre = _masked_pre(op).to(dtype)
    weight = (u * op.scale_post.to(dtype).reshape(-1, 1)) @ (
        v * op.scale_mid.to(dtype).reshape(-1, 1) * pre.reshape(1, -1)
    )
    sal = _salient_weights(op)
    if sal is not None and op.outlier_indices is not None:
        weight[:, op.outlier_indices.long()] += sal.to(dtype)
    if op.patch_left is not None and op.patch_right is not None:
        weight = weight + op.patch_left.to(dtype) @ op.patch_right.to(dtype)
    bias = None if op.bias is None else op.bias.to(dtype)
    return F.linear(value.to(dtype), weight, bias)


def relative_l2(actual: torch.Tensor, expected: torch.Tensor) -> float:
    """``||a - e||_2 / ||e||_2`` in float64."""

    a = actual.detach().double().cpu()
    e = expected.detach().double().cpu()
    denom = float(torch.linalg.vector_norm(e))
    num = float(torch.linalg.vector_norm(a - e))
    return num / denom if denom > 0 else num


def row_sidecar_as_patch(
    out_features: int, indices: torch.Tensor, values: torch.Tensor, scales: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor]:
    """An output-row int8 sidecar as the reference's float patch
    (src/nanoquant/runtime/reference.py:224-233): ``patch_left[idx_k, k] = scale_k``,
    ``patch_right[k] = float(row_k)``."""

    k = int(indices.numel())
    left = torch.zeros(out_features, k, dtype=torch.float32)
    left[indices.long(), torch.arange(k)] = scales.float()
    return left, values.float()


def operands_from_state(state) -> PackedOperands:
    """Read a packed layer's tensors by role (duck-typed on the reference's
    ``PackedLayerState`` field names; an output-row sidecar state is folded in
    as its float patch). Everything is copied to the host."""

    base = getattr(state, "base", state)
    spec = base.spec

    def host(t):
        return None if t is None else t.detach().cpu()

    patch_left, patch_right = host(base.patch_left), host(base.patch_right)
    rows = getattr(state, "rows", None)
    if rows is not None:
        patch_left, patch_right = row_sidecar_as_patch(
            spec.out_features, host(rows.indices), host(rows.values), host(rows.scales)
        )
    return PackedOperands(
        spec.in_features,
        spec.out_features,
        spec.rank,
        host(base.left_words).numpy(),
        host(base.right_words).numpy(),
        host(base.scale_pre),
        host(base.scale_mid),
        host(base.scale_post),
        host(base.bias),
        host(base.outlier_indices),
        host(base.outlier_values),
        host(base.outlier_scales),
        patch_left,
        patch_right,
    )
