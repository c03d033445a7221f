"""Host-side runtime API: layout helpers, layer-state invariants, capability
codes, backend selection and the module binding, with fake backends; no GPU
needed. The layout and state cases follow the reference's
tests/unit/test_runtime_{packed,backend}.py."""

from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest
import torch
from torch import nn

from nanoquant_amd.runtime import (
    GGUF_TENSOR_SUFFIXES,
    PACKED_LAYOUT_VERSION,
    PACKED_REFERENCE_COMMIT,
    PACKED_REFERENCE_CUDA_SHA256,
    BackendCapabilities,
    HipPackedBackend,
    LogicalLayerState,
    PackedLayerState,
    PackedLayoutMetadata,
    PreparedLayer,
    PreparedLinear,
    PreparedModel,
    QuantizedLinearSpec,
    SelectionError,
    SupportResult,
    WorkloadSpec,
    bind_prepared_linears,
    evaluate_capabilities,
    execution_workload,
    pack_logical_layer,
    pack_sign_matrix,
    packed_row_stride_bytes,
    choose_backends,
    packed_word_count,
    prepare_hip_projection_group,
    supports_vector_word_loads,
    unpack_sign_matrix,
)
from nanoquant_amd.runtime import _native
from nanoquant_amd.synthetic import qwen3_8b_layer, synthetic_packed_layer, synthetic_row_sidecar
from oracle import nq_oracle as orc

# --- layout ----------------------------------------------------------------------


@pytest.mark.parametrize("columns", (1, 31, 32, 33, 65, 128))
def test_host_pack_unpack_is_bit_exact_with_oracle(columns):
    values = torch.where(torch.arange(3 * columns).reshape(3, columns) % 3 == 0, -1.0, 1.0)
    packed = pack_sign_matrix(values)
    assert packed.dtype == torch.int32 and packed.shape == (3, packed_word_count(columns))
    assert np.array_equal(packed.numpy(), orc.pack_signs(values.numpy().astype(np.int8)))
    assert torch.equal(unpack_sign_matrix(packed, 3, columns), values)


def test_host_pack_known_answer_words():
    values = torch.ones(2, 32)
    values[0, (0, 1, 31)] = -1
    values[1] = -1
    packed = pack_sign_matrix(values)
    assert int(packed[0, 0]) == -(2**31) + 3
    assert int(packed[1, 0]) == -1


def test_host_unpack_rejects_padding():
    packed = pack_sign_matrix(torch.ones(1, 33))
    packed[0, -1] = 2
    with pytest.raises(ValueError, match="non-zero padding bit"):
        unpack_sign_matrix(packed, 1, 33)


def test_row_stride_and_vector_predicate():
    assert packed_row_stride_bytes(33) == 8
    assert packed_row_stride_bytes(128) == 16
    assert not supports_vector_word_loads(pack_sign_matrix(torch.ones(2, 33)))
    assert supports_vector_word_loads(pack_sign_matrix(torch.ones(2, 128)))


def test_layout_metadata_contract():
    layout = PackedLayoutMetadata()
    assert layout.version == "llama.cpp-i32-lsb-v1" == PACKED_LAYOUT_VERSION
    assert (layout.positive_bit, layout.negative_bit, layout.padding_bit) == (0, 1, 0)
    assert layout.bit_order == "least-significant-bit-first"
    assert (layout.right_sidecar_name, layout.left_sidecar_name) == ("nq_v", "nq_u")
    assert dict(GGUF_TENSOR_SUFFIXES)["outlier_scales"] == "nq_salient_scale"
    assert layout.reference.commit == PACKED_REFERENCE_COMMIT
    assert layout.reference.cuda_sha256 == PACKED_REFERENCE_CUDA_SHA256
    with pytest.raises(ValueError, match="bit order"):
        PackedLayoutMetadata(bit_order="most-significant-bit-first")


# --- layer state -----------------------------------------------------------------


def _logical(factor_dtype=torch.float32) -> LogicalLayerState:
    spec = QuantizedLinearSpec(
        "blocks.0.linear", "nanoquant-v1", 35, 3, 33,
        str(factor_dtype).removeprefix("torch."), "float32",
        outlier_count=2, outlier_value_dtype="int8", has_outlier_scales=True, has_bias=True,
    )
    left = torch.where(torch.arange(99).reshape(3, 33) % 2 == 0, 1.0, -1.0).to(factor_dtype)
    right = torch.where(torch.arange(33 * 35).reshape(33, 35) % 5 == 0, -1.0, 1.0).to(factor_dtype)
    return LogicalLayerState(
        spec, left, right,
        torch.cat((torch.tensor([0.5, 0.0]), torch.linspace(0.5, 1.5, 32), torch.zeros(1))),
        torch.linspace(0.75, 1.25, 33), torch.linspace(1.0, 1.5, 3), torch.tensor([0.1, -0.2, 0.3]),
        torch.tensor([1, 34], dtype=torch.int32),
        torch.tensor([[1, -2], [3, -4], [5, -6]], dtype=torch.int8), torch.tensor([0.25, 0.5]),
    )


@pytest.mark.parametrize("factor_dtype", (torch.float16, torch.bfloat16, torch.float32))
def test_packed_round_trip_preserves_logical_state(factor_dtype):
    logical = _logical(factor_dtype)
    packed = pack_logical_layer(logical)
    restored = packed.to_logical()
    assert packed.left_words.shape == (3, 2) and packed.right_words.shape == (33, 2)
    for a, b in ((logical.left_binary, restored.left_binary), (logical.right_binary, restored.right_binary),
                 (logical.scale_pre, restored.scale_pre), (logical.outlier_values, restored.outlier_values)):
        assert torch.equal(a, b)


def test_packed_state_rejects_nonzero_scale_pre_at_salient_column():
    logical = _logical()
    pre = logical.scale_pre.clone()
    pre[1] = 1
    with pytest.raises(ValueError, match="exactly zero scale_pre"):
        PackedLayerState(
            logical.spec, PACKED_LAYOUT_VERSION, pack_sign_matrix(logical.left_binary),
            pack_sign_matrix(logical.right_binary), pre, logical.scale_mid, logical.scale_post,
            logical.bias, logical.outlier_indices, logical.outlier_values, logical.outlier_scales,
        )


def test_packed_state_rejects_scales_on_float_salient_values():
    packed = pack_logical_layer(_logical())
    with pytest.raises(ValueError, match="scales require int8"):
        PackedLayerState(
            replace(packed.spec, outlier_value_dtype="float32"), packed.layout, packed.left_words,
            packed.right_words, packed.scale_pre, packed.scale_mid, packed.scale_post, packed.bias,
            packed.outlier_indices, packed.outlier_values.float(), packed.outlier_scales,
        )


def test_logical_state_rejects_non_sign_and_unsorted_outliers():
    state = _logical()
    bad = state.left_binary.clone()
    bad[0, 0] = 0
    with pytest.raises(ValueError, match=r"other than -1 or \+1"):
        LogicalLayerState(state.spec, bad, state.right_binary, state.scale_pre, state.scale_mid,
                          state.scale_post, state.bias, state.outlier_indices, state.outlier_values,
                          state.outlier_scales)
    with pytest.raises(ValueError, match="strictly increasing"):
        LogicalLayerState(state.spec, state.left_binary, state.right_binary, state.scale_pre,
                          state.scale_mid, state.scale_post, state.bias,
                          torch.tensor([34, 1], dtype=torch.int32), state.outlier_values,
                          state.outlier_scales)


def test_row_sidecar_state_folds_into_reference_patch():
    shape = qwen3_8b_layer()[1]
    small = replace(shape, in_features=96, out_features=40, rank=19)
    base = synthetic_packed_layer(small, seed=1)
    state = synthetic_row_sidecar(base, 4, seed=2)
    logical = state.to_logical()
    assert logical.spec.patch_rank == 4 and logical.patch_left.shape == (40, 4)
    x = torch.randn(2, 96)
    op = orc.operands_from_state(state)
    direct = orc.packed_forward(orc.operands_from_state(base), x, dtype=torch.float64)
    rows = state.rows
    direct.index_add_(1, rows.indices.long(), (x.double() @ rows.values.double().T) * rows.scales.double())
    torch.testing.assert_close(orc.packed_forward(op, x, dtype=torch.float64), direct)


# --- capabilities and planning -----------------------------------------------------


def _spec(name="blocks.0.mlp.proj") -> QuantizedLinearSpec:
    return QuantizedLinearSpec(name, "nanoquant-v1", 4, 3, 2, "float32", "float32",
                               outlier_count=1, outlier_value_dtype="int8",
                               has_outlier_scales=True, has_bias=True)


def test_capability_first_failure_is_stable():
    caps = BackendCapabilities(
        logical_formats=("nanoquant-v1",), device_types=("cuda",), input_dtypes=("bfloat16",),
        factor_dtypes=("float32",), scale_dtypes=("float32",), outlier_value_dtypes=("int8",),
        workload_kinds=("decode",), supports_bias=True, supports_outliers=True,
        supports_deterministic=True, in_feature_alignment=8,
    )
    op = QuantizedLinearSpec("blocks.0.attn.q_proj", "nanoquant-v1", 12, 8, 8, "float32", "float32")
    work = WorkloadSpec("decode", "cuda", "bfloat16", 1, 1, deterministic=True)
    assert evaluate_capabilities(caps, op, work) == SupportResult.rejected(
        "NQ-INF-IN-ALIGNMENT", "input features must be aligned to 8")
    assert evaluate_capabilities(caps, op, replace(work, kind="prefill")).code == "NQ-INF-WORKLOAD"
    assert evaluate_capabilities(caps, replace(op, logical_format="x"), work).code == "NQ-INF-FORMAT"


def test_hip_backend_reports_missing_device_and_library(monkeypatch):
    backend = HipPackedBackend()
    work = WorkloadSpec("decode", "cuda", "bfloat16", 1, 1, deterministic=True)
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    assert backend.supports(_spec(), work).code == "NQ-INF-DEVICE-UNAVAILABLE"
    monkeypatch.setattr(_native, "library_available", lambda: False)
    assert backend.supports(_spec(), work).code == "NQ-INF-HIP-KERNEL"
    assert backend.supports(_spec(), replace(work, device_type="cpu")).code == "NQ-INF-DEVICE"


def test_hip_backend_declares_reference_capabilities():
    caps = HipPackedBackend().capabilities()
    assert caps.device_types == ("cuda",)
    assert caps.workload_kinds == ("prefill", "decode")
    assert caps.supports_outliers and caps.supports_bias and caps.supports_deterministic
    assert set(caps.outlier_value_dtypes) == {"float16", "bfloat16", "float32", "int8"}


class _KindBackend:
    version = "1"

    def __init__(self, name, kinds, reject_code=None):
        self.name, self.kinds, self.reject_code = name, kinds, reject_code
        self.prepare_count = 0

    def capabilities(self):
        return HipPackedBackend().capabilities()

    def supports(self, op, workload):
        if self.reject_code:
            return SupportResult.rejected(self.reject_code, "rank must be aligned to 32")
        if workload.kind not in self.kinds:
            return SupportResult.rejected("NQ-INF-WORKLOAD", f"{workload.kind} is not selected")
        return SupportResult.accepted()

    def prepare(self, state, device):
        self.prepare_count += 1
        return PreparedLayer(self.name, self.version, state.spec, state)

    def linear(self, value, layer):
        return torch.zeros(*value.shape[:-1], layer.spec.out_features, dtype=torch.float32)


def _state(name):
    spec = QuantizedLinearSpec(name, "nanoquant-v1", 4, 3, 2, "float32", "float32")
    return LogicalLayerState(spec, torch.tensor([[1.0, -1.0], [-1.0, 1.0], [1.0, 1.0]]),
                             torch.tensor([[1.0, -1.0, 1.0, -1.0], [-1.0, -1.0, 1.0, 1.0]]),
                             torch.ones(4), torch.ones(2), torch.ones(3))


def test_selection_fallback_strict_and_named_rejections():
    states = {n: _state(n) for n in ("blocks.0.proj", "blocks.1.proj")}
    rejecting = _KindBackend("rejecting", ("prefill", "decode"), reject_code="NQ-INF-RANK-ALIGNMENT")
    fallback = _KindBackend("fallback", ("prefill", "decode"))
    work = WorkloadSpec("decode", "cpu", "float32", 1, 1, deterministic=True)
    choices = choose_backends([s.spec for s in states.values()], work, (rejecting, fallback), strict=False)
    assert [c.fallback for c in choices] == [True, True]
    assert [c.rejections[0].code for c in choices] == ["NQ-INF-RANK-ALIGNMENT"] * 2
    assert [c.backend for c in choices] == [fallback, fallback]
    with pytest.raises(SelectionError, match="strict selection refuses the fallback.*NQ-INF-RANK-ALIGNMENT"):
        choose_backends((_spec(),), work, (rejecting, fallback), strict=True)
    with pytest.raises(SelectionError, match="no backend accepts the decode workload.*NQ-INF-RANK-ALIGNMENT"):
        choose_backends((_spec(),), work, (rejecting,), strict=False)
    with pytest.raises(ValueError, match="unique"):
        choose_backends((_spec(), _spec()), work, (fallback,), strict=False)


def _model(states, backend, *, batch=2, prefill_tokens=3, device="cpu"):
    return PreparedModel(
        states,
        prefill=WorkloadSpec("prefill", "cpu", "float32", batch, prefill_tokens, deterministic=True),
        decode=WorkloadSpec("decode", "cpu", "float32", batch, 1, deterministic=True),
        backends=(backend,), device=device,
    )


def test_prepared_model_shares_payloads_and_fixes_decode_geometry():
    states = {n: _state(n) for n in ("blocks.0.proj", "blocks.1.proj")}
    backend = _KindBackend("both", ("prefill", "decode"))
    model = _model(states, backend)
    assert backend.prepare_count == 2
    assert all(model.prepared("prefill", i) is model.prepared("decode", i) for i in range(2))
    assert model.linear("prefill", 0, torch.ones(2, 1, 4)).shape == (2, 1, 3)
    with pytest.raises(ValueError, match="prefill input holds 8 token slots; at most 6 fit"):
        model.linear("prefill", 0, torch.ones(2, 4, 4))
    with pytest.raises(ValueError, match="decode input holds 6 token slots; it must hold 2"):
        model.linear("decode", 0, torch.ones(2, 3, 4))
    with pytest.raises(ValueError, match="prefill input dtype"):
        model.linear("prefill", 0, torch.ones(2, 3, 4, dtype=torch.float16))
    with pytest.raises(IndexError, match="not in the inventory"):
        model.linear("decode", 2, torch.ones(2, 4))
    with pytest.raises(ValueError, match="decode workload runs one token"):
        PreparedModel(states, prefill=WorkloadSpec("prefill", "cpu", "float32", 1, 4),
                      decode=WorkloadSpec("decode", "cpu", "float32", 1, 2), backends=(backend,), device="cpu")
    with pytest.raises(ValueError, match="is not the preparation device 'cuda'"):
        _model(states, backend, device="cuda")
    with pytest.raises(ValueError, match="stored under the name"):
        _model({"blocks.9.proj": states["blocks.0.proj"]}, backend)


def test_prepared_linear_binding_and_context():
    states = {"blocks.0.mlp.up": _state("blocks.0.mlp.up")}
    backend = _KindBackend("both", ("prefill", "decode"))
    prepared = _model(states, backend, batch=1, prefill_tokens=4)
    model = nn.Module()
    model.mlp = nn.Module()
    model.mlp.up = nn.Linear(4, 3)
    assert bind_prepared_linears(model, prepared, {"blocks.0.mlp.up": "mlp.up"}) == 1
    assert isinstance(model.mlp.up, PreparedLinear)
    with pytest.raises(RuntimeError, match="outside an execution_workload"):
        model.mlp.up(torch.ones(1, 4))
    with execution_workload("decode"):
        assert model.mlp.up(torch.ones(1, 4)).shape == (1, 3)


def test_projection_group_declines_layers_it_cannot_launch_together():
    """prepare_hip_projection_group answers None (the reference's contract for
    an incompatible group) for foreign payloads and wrong member counts."""

    foreign = [PreparedLayer("torch-packed-reference", "1", _spec(f"blocks.0.p{i}"), object()) for i in range(3)]
    assert prepare_hip_projection_group(tuple(foreign)) is None
    assert prepare_hip_projection_group(tuple(foreign[:1])) is None
    assert prepare_hip_projection_group(tuple(foreign * 3)) is None


def test_linear_input_checks_follow_the_reference():
    """HipPackedBackend.linear's input checks, each a ValueError raised before
    any launch (src/nanoquant/runtime/cuda_backend.py:243-260): the layer's
    device, a float dtype, last dimension == in_features, at least one token,
    contiguous, no autograd."""

    from nanoquant_amd.runtime.hip_backend import _check_value

    spec = QuantizedLinearSpec("blocks.0.t", "nanoquant-v1", 8, 3, 4, "float32", "float16")
    cpu = torch.device("cpu")
    for dtype in (torch.float16, torch.bfloat16, torch.float32):
        _check_value(torch.zeros(2, 8, dtype=dtype), spec, cpu)
    _check_value(torch.zeros(3, 2, 8), spec, cpu)
    cases = [
        (torch.zeros(2, 8), torch.device("cuda", 0), "same device"),
        (torch.zeros(2, 8, dtype=torch.int32), cpu, "dtype is unsupported"),
        (torch.zeros(2, 7), cpu, "feature dimension"),
        (torch.tensor(1.0), cpu, "feature dimension"),
        (torch.zeros(0, 8), cpu, "at least one token"),
        (torch.zeros(8, 2).t(), cpu, "contiguous"),
        (torch.zeros(2, 16)[:, ::2], cpu, "contiguous"),
        (torch.zeros(2, 8, requires_grad=True), cpu, "autograd"),
    ]
    for value, device, match in cases:
        with pytest.raises(ValueError, match=match):
            _check_value(value, spec, device)


# --- the reference's own objects (stand-ins with its field names) -------------------


def test_supports_reads_reference_spec_and_workload_objects(monkeypatch):
    """``supports`` gives a spec and workload of another class (the
    reference's field names, src/nanoquant/runtime/backend.py:27-91) the same
    codes as this package's own, in the reference's order."""

    from foreign_state import ForeignWorkload, foreign_spec

    backend = HipPackedBackend()
    own_work = WorkloadSpec("decode", "cuda", "bfloat16", 1, 1, deterministic=True)
    work = ForeignWorkload("decode", "cuda", "bfloat16", 1, 1, deterministic=True)
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    cases = [
        (_spec(), work),
        (_spec(), replace(work, device_type="cpu")),
        (_spec(), replace(work, input_dtype="int8")),
        (replace(_spec(), logical_format="x"), work),
        (replace(_spec(), factor_dtype="float64"), work),
        (replace(_spec(), outlier_value_dtype="float64"), work),
        (_spec(), replace(work, kind="prefill", token_count=64)),
    ]
    codes = []
    for spec, workload in cases:
        own = backend.supports(spec, WorkloadSpec(**{k: getattr(workload, k) for k in WorkloadSpec.__slots__}))
        got = backend.supports(foreign_spec(spec), workload)
        assert got == own
        codes.append(got.code)
    assert codes == ["NQ-INF-DEVICE-UNAVAILABLE", "NQ-INF-DEVICE", "NQ-INF-INPUT-DTYPE", "NQ-INF-FORMAT",
                     "NQ-INF-FACTOR-DTYPE", "NQ-INF-OUTLIER-DTYPE", "NQ-INF-DEVICE-UNAVAILABLE"]
    monkeypatch.setattr(_native, "library_available", lambda: False)
    assert backend.supports(foreign_spec(_spec()), work).code == "NQ-INF-HIP-KERNEL"
    assert own_work.kind == work.kind


def test_prepare_accepts_reference_state_objects():
    """A state of another class with the reference's field names
    (src/nanoquant/runtime/packed.py:231-244) passes the backend's type
    check: on a CPU device ``prepare`` stops at the device check, as for this
    package's own state. The adopted state keeps the caller's spec object,
    which the reference planner compares with the prepared layer's spec
    (src/nanoquant/runtime/planning.py:255-256)."""

    from foreign_state import ForeignPackedLayerState, foreign_copy
    from nanoquant_amd.runtime.hip_backend import adopt_layer_state

    state = synthetic_packed_layer(qwen3_8b_layer()[1], seed=5)
    foreign = foreign_copy(state)
    assert not isinstance(foreign, PackedLayerState) and not isinstance(foreign.spec, QuantizedLinearSpec)
    backend = HipPackedBackend()
    for candidate in (state, foreign):
        with pytest.raises(ValueError, match="requires a CUDA"):
            backend.prepare(candidate, "cpu")
    adopted = adopt_layer_state(foreign)
    assert isinstance(adopted, PackedLayerState) and adopted.spec is foreign.spec
    for name in ("left_words", "right_words", "scale_pre", "scale_mid", "scale_post"):
        assert getattr(adopted, name) is getattr(foreign, name)
    assert adopt_layer_state(state) is state
    # an object without the reference's fields is still refused by type
    for bad in (object(), {"spec": foreign.spec}, state.spec):
        with pytest.raises(TypeError, match="requires PackedLayerState"):
            backend.prepare(bad, "cpu")
    # the invariants are checked again on adoption: s_in must be 0 at a salient column
    salient = synthetic_packed_layer(qwen3_8b_layer()[1], seed=5, salient=3)
    broken = foreign_copy(salient)
    pre = broken.scale_pre.clone()
    pre[int(broken.outlier_indices[0])] = 1.0
    broken = ForeignPackedLayerState(**{**{k: getattr(broken, k) for k in broken.__slots__}, "scale_pre": pre})
    with pytest.raises(ValueError, match="salient"):
        adopt_layer_state(broken)


def test_prepare_accepts_reference_mixed_v_state_objects():
    """A mixed-V state of another class (src/nanoquant/runtime/mixed_v.py:169-187)
    is adopted as this package's MixedVLayerState and expands to the same
    packed words."""

    from foreign_state import ForeignMixedVLayerState, foreign_copy
    from nanoquant_amd.runtime.codecs import MixedVLayerState
    from nanoquant_amd.runtime.hip_backend import adopt_layer_state

    from test_codecs import _mixed_fixture

    state = _mixed_fixture()[0]
    foreign = foreign_copy(state, ForeignMixedVLayerState)
    adopted = adopt_layer_state(foreign)
    assert isinstance(adopted, MixedVLayerState) and adopted.spec is foreign.spec
    assert torch.equal(adopted.to_packed().right_words, state.to_packed().right_words)
    with pytest.raises(ValueError, match="requires a CUDA"):
        HipPackedBackend().prepare(foreign, "cpu")
