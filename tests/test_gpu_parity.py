"""HIP parity against the CPU oracle (run on an MI355X: ``pytest -m gpu``).

Bar: bit-exact for unpacked signs and the GPU tile layout; fp outputs within
the reference tests' ``rtol=2e-5, atol=2e-4`` on the small fixtures (general
fp32 path) and within relative L2 2e-3 of the oracle's fp32 forward for the
tiled MFMA paths; bit-exact replay.
"""

from __future__ import annotations

import json
import sys
from dataclasses import replace
from itertools import product
from pathlib import Path

import numpy as np
import pytest
import torch

from nanoquant_amd import synthetic as syn
from nanoquant_amd.runtime import (
    HipPackedBackend,
    LogicalLayerState,
    PreparedLinear,
    PreparedModel,
    QuantizedLinearSpec,
    WorkloadSpec,
    execution_workload,
    grouped_hip_projection,
    pack_logical_layer,
    prepare_hip_projection_group,
    pack_sign_matrix,
    unpack_sign_matrix_device,
)
from nanoquant_amd.runtime import _native
from oracle import nq_oracle as orc

from tile_layout import build_tiles, geometry as tile_geometry

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a HIP device"),
]

REL_L2 = 2e-3  # tolerance of the tiled MFMA paths against the fp32 reference forward
GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_fixtures.json").read_text())
_FLOATS = (torch.float16, torch.bfloat16, torch.float32)


def _say(*parts) -> None:
    print("[case]", *parts, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", params=["split", "fused", "general"])
def backend(request) -> HipPackedBackend:
    """``split`` / ``fused``: the tiled MFMA kernels (decode as two kernels or
    as one kernel with an in-kernel handoff; prefill above 16 tokens);
    ``general``: the canonical-word fp32 path used for every token count."""

    if request.param == "general":
        return HipPackedBackend(tiled_decode=False)
    return HipPackedBackend(decode_launch=request.param)


def _tiled(backend) -> bool:
    return backend._tiled_decode


def _assert_parity(backend, actual, expected, case=None):
    """fp32 path: the reference tests' rtol=2e-5/atol=2e-4. Tiled MFMA paths
    (int8 decode, fp16 prefill): relative L2 <= 2e-3 against the fp32
    forward."""

    if _tiled(backend):
        err = orc.relative_l2(actual, expected)
        assert err <= REL_L2, (case, err)
    else:
        torch.testing.assert_close(actual.cpu(), expected.float(), rtol=2e-5, atol=2e-4,
                                   msg=lambda m: f"{case}: {m}")


def _sync_header_clean(layer) -> bool:
    """The decode sync header's last line holds the sticky timeout flag (word 0,
    must be 0: no launch ever timed out waiting for stage 1) and the magic."""

    tiles = layer.payload.tiles
    if tiles is None:
        return True
    torch.cuda.synchronize()
    size = int(_native.load().nq_tiles_header_bytes())
    misc = tiles[:size].view(torch.int32).cpu()[-64:]
    return int(misc[0]) == 0 and int(misc[1]) == 0x4E515433


def _run(backend, state, x):
    layer = backend.prepare(state, "cuda")
    return backend.linear(x.cuda(), layer), layer


# --- tile layout ---------------------------------------------------------------------


@pytest.mark.parametrize("inp,out,rank", [(128, 16, 16), (819, 33, 100), (4096, 1024, 819), (1152, 6912, 768),
                                         (12288, 40, 3072), (5, 3, 7)])
def test_prepared_tiles_match_layout(inp, out, rank):
    """nq_prepare_tiles writes V and U in the documented layout, word for word."""

    _say("tiles", inp, out, rank)
    shape = syn.LinearShape("t", inp, out, rank)
    state = syn.synthetic_packed_layer(shape, seed=11)
    layer = HipPackedBackend().prepare(state, "cuda")
    torch.cuda.synchronize()
    header = int(_native.load().nq_tiles_header_bytes()) // 4
    words = layer.payload.tiles.view(torch.int32).cpu().numpy().view(np.uint32)
    nt1, nb1, _ = tile_geometry(rank, inp)
    nt2, nb2, _ = tile_geometry(out, rank)
    v = words[header:header + nt1 * nb1 * 64]
    u = words[header + nt1 * nb1 * 64:header + nt1 * nb1 * 64 + nt2 * nb2 * 64]
    np.testing.assert_array_equal(v, build_tiles(state.right_words.numpy(), rank, inp))
    np.testing.assert_array_equal(u, build_tiles(state.left_words.numpy(), out, rank))


# --- unpack ------------------------------------------------------------------------


@pytest.mark.parametrize("rows,cols", [(3, 1), (3, 31), (2, 32), (5, 33), (4, 65), (819, 4096), (3072, 819)])
@pytest.mark.parametrize("dtype", _FLOATS)
def test_device_unpack_bit_exact(rows, cols, dtype):
    _say("unpack", rows, cols, dtype)
    g = torch.Generator().manual_seed(rows * 7 + cols)
    signs = torch.where(torch.rand(rows, cols, generator=g) < 0.5, -1.0, 1.0)
    words = pack_sign_matrix(signs)
    out = unpack_sign_matrix_device(words.cuda(), rows, cols, dtype=dtype)
    expected = orc.unpack_signs(words.numpy(), rows, cols)
    assert out.dtype == dtype
    assert np.array_equal(out.float().cpu().numpy(), expected.astype(np.float32))
    # Bit patterns, not just values: +1 / -1 exactly.
    assert torch.equal(out.cpu(), torch.from_numpy(expected).to(dtype))


def test_device_unpack_rejects_padding():
    words = pack_sign_matrix(torch.ones(4, 33))
    words[2, -1] = 2
    with pytest.raises(ValueError, match="non-zero padding bit"):
        unpack_sign_matrix_device(words.cuda(), 4, 33)


# --- reference fixtures ----------------------------------------------------------------


def test_golden_fixture_on_gpu(backend):
    f = next(f for f in GOLDEN["fixtures"] if f["name"].startswith("packed_35x3"))
    _say("golden", f["name"])
    spec = QuantizedLinearSpec("blocks.0.linear", "nanoquant-v1", 35, 3, 33, "float32", "float32",
                               outlier_count=2, outlier_value_dtype="int8",
                               has_outlier_scales=True, has_bias=True)
    logical = LogicalLayerState(
        spec,
        torch.tensor(f["left"], dtype=torch.float32),
        torch.tensor(f["right"], dtype=torch.float32),
        torch.tensor(f["scale_pre"], dtype=torch.float32),
        torch.tensor(f["scale_mid"], dtype=torch.float32),
        torch.tensor(f["scale_post"], dtype=torch.float32),
        torch.tensor(f["bias"], dtype=torch.float32),
        torch.tensor(f["outlier_indices"], dtype=torch.int32),
        torch.tensor(f["outlier_values"], dtype=torch.int8),
        torch.tensor(f["outlier_scales"], dtype=torch.float32),
    )
    packed = pack_logical_layer(logical)
    assert packed.left_words.tolist() == f["left_words"]
    y, layer = _run(backend, packed, torch.tensor(f["x"], dtype=torch.float32))
    _assert_parity(backend, y, torch.tensor(f["expected_y"], dtype=torch.float64), f["name"])
    assert _sync_header_clean(layer)


def _matrix_state(factor_dtype, scale_dtype, outlier_dtype, bias) -> LogicalLayerState:
    """35->17, rank 33 word-tail geometry with salient columns {0, 17, 34}
    (geometry of tests/unit/test_runtime_cuda_matrix.py:37-113)."""

    in_f, out_f, rank = 35, 17, 33
    count = 0 if outlier_dtype is None else 3
    spec = QuantizedLinearSpec(
        "blocks.0.self_attn.q_proj", "nanoquant-v1", in_f, out_f, rank,
        str(factor_dtype).removeprefix("torch."), str(scale_dtype).removeprefix("torch."),
        outlier_count=count,
        outlier_value_dtype=None if outlier_dtype is None else str(outlier_dtype).removeprefix("torch."),
        has_outlier_scales=outlier_dtype is torch.int8, has_bias=bias,
    )
    g = torch.Generator().manual_seed(20260715)
    left = torch.where(torch.rand(out_f, rank, generator=g) > 0.5, 1.0, -1.0).to(factor_dtype)
    right = torch.where(torch.rand(rank, in_f, generator=g) > 0.5, 1.0, -1.0).to(factor_dtype)
    pre = torch.randn(in_f, generator=g).to(scale_dtype)
    idx = torch.tensor((0, 17, 34), dtype=torch.int32) if count else None
    if idx is not None:
        pre[idx.long()] = 0
    if outlier_dtype is None:
        values = None
    elif outlier_dtype is torch.int8:
        values = torch.randint(-8, 8, (out_f, count), generator=g, dtype=torch.int8)
    else:
        values = torch.randn(out_f, count, generator=g).to(outlier_dtype)
    return LogicalLayerState(
        spec, left, right, pre,
        torch.randn(rank, generator=g).to(scale_dtype),
        torch.randn(out_f, generator=g).to(scale_dtype),
        bias=torch.randn(out_f, generator=g).to(scale_dtype) if bias else None,
        outlier_indices=idx, outlier_values=values,
        outlier_scales=torch.tensor((0.125, 0.25, 0.375), dtype=scale_dtype) if outlier_dtype is torch.int8 else None,
    )


def test_full_dtype_salient_workload_matrix(backend):
    """Every factor x scale x salient x bias x input dtype x workload combination."""

    executed = 0
    for factor, scale, outlier, bias in product(_FLOATS, _FLOATS, (None, *_FLOATS, torch.int8), (False, True)):
        logical = _matrix_state(factor, scale, outlier, bias)
        packed = pack_logical_layer(logical)
        layer = backend.prepare(packed, "cuda:0")
        oracle_fwd = orc.CpuPackedForward(orc.operands_from_state(packed))
        for input_dtype, kind in product(_FLOATS, ("prefill", "decode")):
            shape = (2, 3) if kind == "prefill" else (2,)
            work = WorkloadSpec(kind, "cuda", str(input_dtype).removeprefix("torch."), 2,
                                3 if kind == "prefill" else 1, deterministic=True)
            assert backend.supports(packed.spec, work).supported
            x = torch.linspace(-0.75, 0.875, 35 * (6 if kind == "prefill" else 2), dtype=input_dtype)
            x = x.reshape(*shape, 35)
            actual = backend.linear(x.cuda(), layer)
            repeated = backend.linear(x.cuda(), layer)
            case = (factor, scale, outlier, bias, input_dtype, kind)
            assert actual.dtype == torch.float32
            _assert_parity(backend, actual, oracle_fwd(x), case)
            assert torch.equal(actual, repeated), case
            executed += 1
        assert _sync_header_clean(layer)
    assert executed == 540


def test_more_than_one_salient_tile_and_patch(backend):
    logical = _matrix_state(torch.float32, torch.float32, torch.float32, False)
    g = torch.Generator().manual_seed(99)
    spec = replace(logical.spec, outlier_count=33, patch_rank=2, patch_value_dtype="float32")
    idx = torch.arange(33, dtype=torch.int32)
    pre = logical.scale_pre.clone()
    pre[:33] = 0
    state = LogicalLayerState(
        spec, logical.left_binary, logical.right_binary, pre, logical.scale_mid, logical.scale_post,
        None, idx, torch.randn(17, 33, generator=g), None,
        torch.randn(17, 2, generator=g), torch.randn(2, 35, generator=g),
    )
    packed = pack_logical_layer(state)
    x = torch.linspace(-0.5, 0.75, 70, dtype=torch.float32).reshape(2, 35)
    y, _ = _run(backend, packed, x)
    _assert_parity(backend, y, orc.packed_forward(orc.operands_from_state(packed), x))


@pytest.mark.parametrize("shape", [(32, 16, 24, 1, 0), (33, 17, 25, 1, 3), (64, 32, 48, 4, 4),
                                   (64, 32, 48, 8, 2), (96, 64, 64, 8, 7)])
def test_llama_cpp_backend_ops_cases(backend, shape):
    """Shapes of the llama.cpp test-backend-ops NanoQuant cases with their
    deterministic F16 salient weights ((o*5 + s*3) % 19 - 9) / 128."""

    in_f, rank, out_f, cols, k = shape
    _say("backend-ops", shape)
    base = syn.synthetic_packed_layer(syn.LinearShape("blocks.0.t", in_f, out_f, rank), seed=sum(shape),
                                      salient=k, salient_dtype=torch.float16 if k else None)
    if k:
        o = torch.arange(out_f).reshape(-1, 1)
        s = torch.arange(k).reshape(1, -1)
        values = (((o * 5 + s * 3) % 19 - 9) * 0.0078125).to(torch.float16)
        base = replace(base, outlier_values=values.contiguous())
    x = syn.synthetic_activations(cols, in_f, seed=1, dtype=torch.float32)
    y, _ = _run(backend, base, x)
    _assert_parity(backend, y, orc.packed_forward(orc.operands_from_state(base), x), shape)


# --- benchmark shapes ----------------------------------------------------------------


def _check_shape(backend, state, tokens, seed, bound=REL_L2):
    x = syn.synthetic_activations(tokens, state.spec.in_features, seed=seed)
    layer = backend.prepare(state, "cuda")
    y = backend.linear(x.cuda(), layer)
    y2 = backend.linear(x.cuda(), layer)
    expected = orc.packed_forward(orc.operands_from_state(state), x)
    err = orc.relative_l2(y, expected)
    assert err <= bound, (state.spec.name, tokens, err)
    assert torch.equal(y, y2)
    assert _sync_header_clean(layer)
    print(f"  {state.spec.name} M={tokens} rel_l2={err:.2e}", flush=True)
    return err


def test_gemma3_1b_gate_decode(backend):
    shape = syn.gemma3_1b_gate()
    _say("gemma gate", shape)
    state = syn.synthetic_packed_layer(shape, seed=syn.BASE_SEED + 0)
    _check_shape(backend, state, 1, seed=1)


@pytest.mark.parametrize("tokens", [1, 4, 16])
def test_qwen3_8b_layer_decode(backend, tokens):
    for i, shape in enumerate(syn.qwen3_8b_layer()):
        _say("qwen", shape.name, tokens)
        state = syn.synthetic_packed_layer(shape, seed=syn.BASE_SEED + 1 + i)
        _check_shape(backend, state, tokens, seed=tokens + i)


@pytest.mark.parametrize("tokens", [64])
def test_llama3_8b_prefill(backend, tokens):
    for i, shape in enumerate(syn.llama3_8b_layer()):
        _say("llama", shape.name, tokens)
        state = syn.synthetic_packed_layer(shape, seed=syn.BASE_SEED + 2 + i)
        _check_shape(backend, state, tokens, seed=tokens + i)


@pytest.mark.parametrize("tokens", [1, 8])
def test_gemma3_4b_down_with_sidecars(backend, tokens):
    shape = syn.gemma3_4b_down()
    _say("gemma down sidecars", tokens)
    column = syn.synthetic_packed_layer(shape, seed=syn.BASE_SEED + 3, salient=26, bias=True)
    _check_shape(backend, column, tokens, seed=tokens)
    plain = syn.synthetic_packed_layer(shape, seed=syn.BASE_SEED + 3)
    rows = syn.synthetic_row_sidecar(plain, 26, seed=syn.BASE_SEED + 4)
    _check_shape(backend, rows, tokens, seed=tokens)


# --- prefill: tokens > 16 run two MFMA sign GEMMs ------------------------------------


@pytest.mark.parametrize("tokens", [17, 40, 129, 300])
@pytest.mark.parametrize("geometry", [(35, 17, 33, 3), (200, 130, 129, 5), (1152, 864, 768, 0),
                                      (640, 257, 96, 31)])
def test_prefill_ragged_geometries(tokens, geometry):
    """Word tails, partial 16-row tiles, partial 128-token blocks, salient
    columns (int8 with scales) and bias on the MFMA prefill kernels."""

    in_f, out_f, rank, k = geometry
    backend = HipPackedBackend()
    _say("prefill ragged", geometry, tokens)
    shape = syn.LinearShape("blocks.0.mlp.gate_proj", in_f, out_f, rank)
    state = syn.synthetic_packed_layer(shape, seed=tokens + sum(geometry), salient=k, bias=True)
    _check_shape(backend, state, tokens, seed=tokens)


@pytest.mark.parametrize("geometry", [(1024, 64, 8000, 2), (512, 7990, 300, 0)])
def test_prefill_wide_blocks(geometry):
    """GEMMs that take the 128 x 256 block tile at M = 2048 (512 such blocks:
    one resident round, against two of 128 x 128 blocks): a rank of 8000 puts
    it on the first GEMM (whose last block reaches past the 8064-column padded
    fp16 intermediate), an output of 7990 rows on the second (a partial last
    block and a partial 16-row tile)."""

    in_f, out_f, rank, k = geometry
    backend = HipPackedBackend()
    _say("prefill wide", geometry)
    shape = syn.LinearShape("blocks.0.mlp.gate_proj", in_f, out_f, rank)
    state = syn.synthetic_packed_layer(shape, seed=sum(geometry), salient=k, bias=True)
    _check_shape(backend, state, 2048, seed=7)


@pytest.mark.parametrize("x_dtype", _FLOATS)
def test_prefill_input_dtypes_and_patch(x_dtype):
    logical = _matrix_state(torch.bfloat16, torch.float16, torch.float16, True)
    packed = pack_logical_layer(logical)
    backend = HipPackedBackend()
    _say("prefill dtype", x_dtype)
    layer = backend.prepare(packed, "cuda")
    x = torch.linspace(-2.0, 1.5, 35 * 70, dtype=x_dtype).reshape(2, 35, 35)
    y = backend.linear(x.cuda(), layer)
    assert y.shape == (2, 35, 17) and y.dtype == torch.float32
    err = orc.relative_l2(y, orc.CpuPackedForward(orc.operands_from_state(packed))(x))
    assert err <= REL_L2, (x_dtype, err)
    shape = syn.gemma3_4b_down()
    rows = syn.synthetic_row_sidecar(syn.synthetic_packed_layer(shape, seed=5), 26, seed=6)
    _check_shape(backend, rows, 64, seed=7)


def test_prefill_output_dtypes():
    backend = HipPackedBackend()
    shape = syn.LinearShape("blocks.0.mlp.down_proj", 512, 384, 200)
    state = syn.synthetic_packed_layer(shape, seed=11, salient=4, bias=True)
    layer = backend.prepare(state, "cuda")
    x = syn.synthetic_activations(96, 512, seed=12, device="cuda")
    y32 = backend.linear(x, layer)
    for dtype in (torch.bfloat16, torch.float16):
        _say("prefill out dtype", dtype)
        out = torch.empty(96, 384, dtype=dtype, device="cuda")
        backend.linear_into(x, layer, output_dtype=dtype, out=out)
        torch.testing.assert_close(out, y32.to(dtype), rtol=0, atol=0)


@pytest.mark.parametrize("tokens", [256, 512, 2048])
def test_llama3_8b_prefill_sweep(tokens):
    """All seven Llama-3-8B linears (q, k, v, o, gate, up, down) against the
    oracle at each token count."""

    backend = HipPackedBackend()
    for i, shape in enumerate(syn.llama3_8b_layer()):
        _say("llama sweep", shape.name, tokens)
        state = syn.synthetic_packed_layer(shape, seed=syn.BASE_SEED + 60 + tokens + i)
        _check_shape(backend, state, tokens, seed=tokens + i)


# Split prefill operands (fp16 value plus fp16 remainder): about 22 bits per
# operand, so the result is within fp32 accumulation error of the oracle's
# fp32 forward (observed about 1e-6).
SPLIT_REL_L2 = 2e-5


@pytest.mark.parametrize("tokens", [17, 64, 300, 512, 2048])
def test_llama3_8b_prefill_split_operands(tokens):
    """The seven Llama-3-8B linears with split prefill operands, every block
    tile (64 x 128 up to 64 tokens, 128 x 128 and 128 x 256 above) and split
    K, against the oracle at SPLIT_REL_L2."""

    backend = HipPackedBackend(prefill_operands="split")
    for i, shape in enumerate(syn.llama3_8b_layer()):
        _say("llama split operands", shape.name, tokens)
        state = syn.synthetic_packed_layer(shape, seed=syn.BASE_SEED + 90 + tokens + i, salient=3 * (i % 2),
                                           bias=i == 6)
        _check_shape(backend, state, tokens, seed=tokens + i, bound=SPLIT_REL_L2)


@pytest.mark.parametrize("tokens", [40, 300])
def test_prefill_split_operands_batch_and_ragged(tokens):
    """A batch of unlike members (generic and vector row passes, word tails,
    split beside unsplit K) with split operands matches the oracle at
    SPLIT_REL_L2 (its K splits are chosen for the whole launch, so members
    need not equal their single calls bit for bit); a batch of one is the
    single call; a batch mixing operand modes is refused."""

    backend = HipPackedBackend(prefill_operands="split")
    shapes = [syn.LinearShape("blocks.0.mlp.gate_proj", 35, 17, 33), syn.LinearShape("blocks.0.mlp.up_proj", 640, 257, 96),
              syn.LinearShape("blocks.0.mlp.down_proj", 4096, 1024, 655)]
    states = [syn.synthetic_packed_layer(sh, seed=tokens + i, salient=2 * i, bias=i == 1) for i, sh in enumerate(shapes)]
    layers = [backend.prepare(st, "cuda") for st in states]
    xs = [syn.synthetic_activations(tokens, sh.in_features, seed=5 + i, device="cuda") for i, sh in enumerate(shapes)]
    _say("split operands batch", tokens)
    outs = backend.linear_batch(xs, layers)
    for st, layer, x, y in zip(states, layers, xs, outs):
        err = orc.relative_l2(y, orc.packed_forward(orc.operands_from_state(st), x.cpu()))
        assert err <= SPLIT_REL_L2, (st.spec.name, err)
        assert torch.equal(backend.linear_batch([x], [layer])[0], backend.linear(x, layer))
    plain = HipPackedBackend().prepare(states[0], "cuda")
    with pytest.raises(_native.NativeCallError):
        backend.linear_batch([xs[0], xs[1]], [plain, layers[1]])


# --- integration ---------------------------------------------------------------------


def test_selection_and_module_on_gpu(backend):
    logical = _matrix_state(torch.float32, torch.bfloat16, torch.bfloat16, True)
    packed = pack_logical_layer(logical)
    prepared = PreparedModel(
        {packed.spec.name: packed},
        prefill=WorkloadSpec("prefill", "cuda", "bfloat16", 1, 4, deterministic=True),
        decode=WorkloadSpec("decode", "cuda", "bfloat16", 1, 1, deterministic=True),
        backends=(backend,), device="cuda",
    )
    assert prepared.prepared("prefill", 0) is prepared.prepared("decode", 0)
    prefill = torch.linspace(-1, 1, 140, dtype=torch.bfloat16).reshape(1, 4, 35).cuda()
    decode = prefill[:, -1, :].contiguous()
    fwd = orc.CpuPackedForward(orc.operands_from_state(packed))
    _assert_parity(backend, prepared.linear("prefill", 0, prefill), fwd(prefill.cpu()))
    _assert_parity(backend, prepared.linear("decode", 0, decode), fwd(decode.cpu()))
    module = PreparedLinear(prepared, 0)
    with execution_workload("decode"):
        out = module(decode)
    assert out.dtype == torch.bfloat16


@pytest.mark.parametrize("tokens", [1, 4, 64])
def test_reference_state_objects_run_through_prepare_and_linear(backend, tokens):
    """States and specs of another class with the reference's field names
    (src/nanoquant/runtime/packed.py:231-244, backend.py:27-73), as the
    reference planner passes them to ``backend.prepare``
    (src/nanoquant/runtime/planning.py:249-257): the prepared layer carries the
    caller's spec, and ``linear`` matches the oracle and, bit for bit, the same
    layer prepared from this package's own state."""

    from foreign_state import foreign_copy

    shape = syn.qwen3_8b_layer()[1]  # k_proj, rank 819 (word tail 19)
    state = syn.synthetic_packed_layer(shape, seed=syn.BASE_SEED + 71, salient=5, salient_dtype=torch.int8,
                                       bias=True)
    foreign = foreign_copy(state)
    _say("foreign state", shape.name, tokens, backend.name)
    layer = backend.prepare(foreign, "cuda")
    assert layer.spec == foreign.spec and layer.spec is foreign.spec
    assert (layer.backend_name, layer.backend_version) == (backend.name, backend.version)
    own = backend.prepare(state, "cuda")
    x = syn.synthetic_activations(tokens, shape.in_features, seed=tokens).cuda()
    y = backend.linear(x, layer)
    assert torch.equal(y, backend.linear(x, own))
    # Workload-sized: rel-L2 against the fp32 forward (the general fp32 path
    # observes about 1e-6 at this size).
    err = orc.relative_l2(y, orc.packed_forward(orc.operands_from_state(foreign), x.cpu()))
    assert err <= (REL_L2 if _tiled(backend) else 1e-5), ("foreign", tokens, err)


def test_hip_graph_capture_replays_match_eager(backend):
    shape = syn.qwen3_8b_layer()[1]
    state = syn.synthetic_packed_layer(shape, seed=7)
    layer = backend.prepare(state, "cuda")
    x = syn.synthetic_activations(1, shape.in_features, seed=3, device="cuda")
    eager = backend.linear(x, layer)
    static_out = torch.empty_like(eager)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        backend.linear_into(x, layer, out=static_out)  # warm the allocator off-graph
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        backend.linear_into(x, layer, out=static_out)
    for _ in range(3):
        static_out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_out, eager)
        _ = backend.linear(x, layer)  # eager work between replays
        torch.cuda.synchronize()


# --- batched launches ----------------------------------------------------------------


@pytest.mark.parametrize("launch", ["split", "fused"])
@pytest.mark.parametrize("tokens", [1, 4, 16])
def test_qkv_and_layer_batches_match_oracle(tokens, launch):
    """One launch for Q/K/V (shared x) and one for all seven Qwen3-8B linears of
    a layer (four distinct inputs); every member against the oracle."""

    backend = HipPackedBackend(decode_launch=launch)
    shapes = syn.qwen3_8b_layer()
    states = [syn.synthetic_packed_layer(s, seed=syn.BASE_SEED + 40 + i) for i, s in enumerate(shapes)]
    layers = [backend.prepare(st, "cuda") for st in states]
    xa = syn.synthetic_activations(tokens, 4096, seed=1, device="cuda")
    xo = syn.synthetic_activations(tokens, 4096, seed=2, device="cuda")
    xm = syn.synthetic_activations(tokens, 4096, seed=3, device="cuda")
    xd = syn.synthetic_activations(tokens, 12288, seed=4, device="cuda")
    inputs = [xa, xa, xa, xo, xm, xm, xd]
    _say("qkv batch", tokens)
    qkv = backend.linear_batch(inputs[:3], layers[:3])
    _say("layer batch", tokens)
    whole = backend.linear_batch(inputs, layers)
    again = backend.linear_batch(inputs, layers)
    for i, (state, x) in enumerate(zip(states, inputs)):
        expected = orc.packed_forward(orc.operands_from_state(state), x.cpu())
        assert orc.relative_l2(whole[i], expected) <= REL_L2, (state.spec.name, tokens)
        assert torch.equal(whole[i], again[i])
        if i < 3:
            assert torch.equal(qkv[i], whole[i])
        single = backend.linear(x, layers[i])
        assert torch.equal(single, whole[i])
    assert all(_sync_header_clean(layer) for layer in layers)


@pytest.mark.parametrize("tokens", [1, 3, 5, 6, 9, 16])
def test_split_and_fused_launches_are_bit_identical(tokens):
    """The two decode launch structures run the same tile arithmetic in the
    same order, so their outputs agree bit for bit (including salient and bias).
    From five tokens the split launch stages x * s_in in a kernel of its own
    (two or four token blocks, two waves per chunk with four) where the fused
    launch stages in every workgroup: the digits, and so the outputs, are the
    same."""

    split, fused = HipPackedBackend(decode_launch="split"), HipPackedBackend(decode_launch="fused")
    for i, shape in enumerate(syn.qwen3_8b_layer()):
        _say("split vs fused", shape.name, tokens)
        state = syn.synthetic_packed_layer(shape, seed=syn.BASE_SEED + 70 + i, salient=3 * i, bias=i % 2 == 1)
        x = syn.synthetic_activations(tokens, shape.in_features, seed=i, device="cuda")
        a = split.linear(x, split.prepare(state, "cuda"))
        b = fused.linear(x, fused.prepare(state, "cuda"))
        assert torch.equal(a, b), shape.name


def test_fused_launch_alternating_grouping_keeps_launch_index():
    """The fused launch derives its launch index from monotonic per-tile arrival
    counters; a layer used alone (one tile per stage-2 workgroup) and inside a
    large batch (two tiles per workgroup), alternately, must stay exact."""

    split, fused = HipPackedBackend(decode_launch="split"), HipPackedBackend(decode_launch="fused")
    shapes = syn.qwen3_8b_layer()
    states = [syn.synthetic_packed_layer(shapes[0], seed=81), syn.synthetic_packed_layer(shapes[4], seed=82)]
    xs = [syn.synthetic_activations(1, 4096, seed=s, device="cuda") for s in (1, 2)]
    ref = [split.linear(x, split.prepare(st, "cuda")) for x, st in zip(xs, states)]
    layers = [fused.prepare(st, "cuda") for st in states]
    for rep in range(4):
        _say("alternating grouping", rep)
        alone = fused.linear(xs[0], layers[0])
        pair = fused.linear_batch(xs, layers)
        assert torch.equal(alone, ref[0]), rep
        assert torch.equal(pair[0], ref[0]) and torch.equal(pair[1], ref[1]), rep
    assert all(_sync_header_clean(layer) for layer in layers)


def test_fused_wait_timeout_poisons_outputs_and_sets_flag():
    """Forced from the host, with every kernel still exiting normally: the
    header's spin limit is lowered to 16 polls and every stage-2 arrival
    counter is advanced by three launches, so no stage-2 workgroup's target
    launch is ever signalled. Each one gives up after 16 polls, stores NaN for
    its outputs and sets the sticky flag."""

    fused = HipPackedBackend(decode_launch="fused")
    shape = syn.qwen3_8b_layer()[1]  # k_proj 4096 -> 1024 r819: 64 stage-2 tiles
    state = syn.synthetic_packed_layer(shape, seed=syn.BASE_SEED + 90)
    layer = fused.prepare(state, "cuda")
    x = syn.synthetic_activations(1, shape.in_features, seed=90, device="cuda")
    good = fused.linear(x, layer)
    assert not fused.fused_launch_timed_out(layer)
    assert orc.relative_l2(good, orc.packed_forward(orc.operands_from_state(state), x.cpu())) <= REL_L2
    # Header lines (256 bytes each; nq_decode_kernels.h): 16 ready slots, the
    # ready root, 32 arrive slots (64-bit counters at the start of lines
    # 17-48), 64 flag replicas, then the misc line (word 3: spin limit).
    header = layer.payload.tiles[: int(_native.load().nq_tiles_header_bytes())]
    lines = header.numel() // 256
    assert lines == 16 + 1 + 32 + 64 + 1
    counters, words = header.view(torch.int64), header.view(torch.int32)
    tiles2 = -(-shape.out_features // 16)
    for slot in range(32):
        participants = tiles2 // 32 + (1 if slot < tiles2 % 32 else 0)
        counters[(17 + slot) * 32] += 3 * participants
    words[(lines - 1) * 64 + 3] = 16
    _say("fused timeout forced", shape.name)
    bad = fused.linear(x, layer)
    torch.cuda.synchronize()
    assert torch.isnan(bad).all()
    assert fused.fused_launch_timed_out(layer)


_PLANTS = (float("nan"), float("inf"), float("-inf"))


def _nonfinite_inputs(tokens: int, width: int, seed: int, first: int = 0) -> torch.Tensor:
    """bf16 activations with NaN, +Inf and -Inf planted at random columns of
    token rows 0, 1, 2 (one token: only row 0, with _PLANTS[first]); with
    more than eight tokens also row 5 (three infinities) and the last row."""

    x = syn.synthetic_activations(tokens, width, seed=seed)
    g = torch.Generator().manual_seed(seed)
    rows = [0] if tokens == 1 else [r for r in (0, 1, 2) if r < tokens - 1]
    for j, t in enumerate(rows):
        x[t, int(torch.randint(0, width, (1,), generator=g))] = _PLANTS[(first + j) % 3]
    if tokens > 8:
        x[5, torch.randint(0, width, (3,), generator=g)] = float("inf")
        x[tokens - 1, int(torch.randint(0, width, (1,), generator=g))] = float("nan")
    return x


@pytest.mark.parametrize("shape_index,tokens,first", [(1, 1, 0), (1, 1, 1), (6, 1, 2), (0, 4, 0), (4, 16, 0)])
def test_nonfinite_activations_poison_their_tokens_decode(backend, shape_index, tokens, first):
    """A NaN or an infinity in a token's activations makes every output of that
    token non-finite (reference.py:208-235 in fp32); the other tokens keep
    their values. Qwen3-8B layer shapes, decode token counts."""

    shape = syn.qwen3_8b_layer()[shape_index]
    _say("nonfinite decode", shape.name, tokens, _PLANTS[first])
    state = syn.synthetic_packed_layer(shape, seed=syn.BASE_SEED + 95 + shape_index, salient=4, bias=True)
    x = _nonfinite_inputs(tokens, shape.in_features, seed=95 + tokens, first=first)
    _check_nonfinite(backend, state, x)


@pytest.mark.parametrize("shape_index,tokens", [(1, 64), (4, 129)])
def test_nonfinite_activations_poison_their_tokens_prefill(backend, shape_index, tokens):
    """Same contract on the prefill path (Llama-3-8B shapes, MFMA GEMMs)."""

    shape = syn.llama3_8b_layer()[shape_index]
    _say("nonfinite prefill", shape.name, tokens)
    state = syn.synthetic_packed_layer(shape, seed=syn.BASE_SEED + 96 + shape_index, salient=4)
    x = _nonfinite_inputs(tokens, shape.in_features, seed=96 + tokens)
    _check_nonfinite(backend, state, x)


def _check_nonfinite(backend, state, x):
    expected = orc.packed_forward(orc.operands_from_state(state), x)
    layer = backend.prepare(state, "cuda")
    actual = backend.linear(x.cuda(), layer).cpu()
    bad_rows = ~torch.isfinite(x.float()).all(dim=1)
    assert bad_rows.any() and (x.shape[0] == 1 or not bad_rows.all())
    assert torch.equal(torch.isfinite(actual), torch.isfinite(expected))
    assert not torch.isfinite(actual[bad_rows]).any()
    if (~bad_rows).any():
        # Full layer shapes: the relative-L2 bar on every path (outputs are
        # sums of thousands of terms, so the small fixtures' elementwise
        # atol does not apply).
        err = orc.relative_l2(actual[~bad_rows], expected[~bad_rows])
        print(f"  finite rows rel_l2={err:.2e}", flush=True)
        assert err <= REL_L2, err


def _group_member(index: int, rank: int, out_features: int) -> LogicalLayerState:
    """A 64-input member with two bf16 salient columns (1 and 7, s_in zero
    there), the geometry of the reference's grouped-projection test
    (tests/unit/test_runtime_cuda_backend.py:152-195, ranks 32/40/48, outputs
    24/16/32)."""

    g = torch.Generator().manual_seed(700 + index)
    spec = QuantizedLinearSpec(f"blocks.0.self_attn.group_{index}", "nanoquant-v1", 64, out_features, rank,
                               "float32", "bfloat16", outlier_count=2, outlier_value_dtype="bfloat16")
    signs = lambda r, c: torch.where(torch.rand(r, c, generator=g) < 0.5, -1.0, 1.0)  # noqa: E731
    left, right = signs(out_features, rank), signs(rank, 64)
    pre = torch.randn(64, generator=g).bfloat16()
    idx = torch.tensor([1, 7], dtype=torch.int32)
    pre[idx.long()] = 0
    return LogicalLayerState(spec, left, right, pre, torch.randn(rank, generator=g).bfloat16(),
                             torch.randn(out_features, generator=g).bfloat16(), outlier_indices=idx,
                             outlier_values=torch.randn(out_features, 2, generator=g).bfloat16())


@pytest.mark.parametrize("group_count", [2, 3])
def test_grouped_projection_entry_points(group_count):
    """prepare_hip_projection_group / grouped_hip_projection: within the
    rel-L2 bar of the oracle, and bit-identical to the same layers run one by
    one and through linear_batch (one launch pair for the group)."""

    backend = HipPackedBackend()
    states = [pack_logical_layer(_group_member(i, r, o)) for i, (r, o) in enumerate([(32, 24), (40, 16), (48, 32)])]
    layers = tuple(backend.prepare(st, "cuda") for st in states[:group_count])
    group = prepare_hip_projection_group(layers)
    assert group is not None and group.ranks == tuple(st.spec.rank for st in states[:group_count])
    value = torch.randn(1, 1, 64, generator=torch.Generator().manual_seed(99)).cuda()
    actual = grouped_hip_projection(value, group)
    assert len(actual) == group_count
    batch = backend.linear_batch([value] * group_count, list(layers))
    for out, layer, state, whole in zip(actual, layers, states, batch):
        assert out.shape == (1, 1, state.spec.out_features) and out.dtype == torch.float32
        assert torch.equal(out, backend.linear(value, layer))
        assert torch.equal(out, whole)
        err = orc.relative_l2(out, orc.packed_forward(orc.operands_from_state(state), value.cpu()))
        assert err <= REL_L2, err
    assert prepare_hip_projection_group(layers[:1]) is None
    assert prepare_hip_projection_group((layers[0], layers[0])) is None


@pytest.mark.parametrize("tokens", [1, 4, 64])
def test_grouped_projection_qwen3_qkv_and_gate_up(tokens):
    """Qwen3-8B Q/K/V (ranks 2048/819/819, which the reference's grouped path
    rejects) and gate/up through the grouped entry points; 64 tokens run each
    member's prefill call."""

    backend = HipPackedBackend()
    shapes = syn.qwen3_8b_layer()
    for members in ((0, 1, 2), (4, 5)):
        states = [syn.synthetic_packed_layer(shapes[i], seed=syn.BASE_SEED + 120 + i) for i in members]
        group = prepare_hip_projection_group(tuple(backend.prepare(st, "cuda") for st in states))
        assert group is not None
        x = syn.synthetic_activations(tokens, 4096, seed=120 + tokens)
        _say("grouped qwen", members, tokens)
        for out, state in zip(grouped_hip_projection(x.cuda(), group), states):
            err = orc.relative_l2(out, orc.packed_forward(orc.operands_from_state(state), x))
            assert err <= REL_L2, (state.spec.name, err)


@pytest.mark.parametrize("tokens", [17, 64, 300])
def test_prefill_batches_match_oracle(tokens):
    """Above 16 tokens a batch runs each prefill phase (row passes, both sign
    GEMMs, their split-K reductions) as one launch for all members, with K
    splits chosen for the whole launch. Q/K/V of Llama-3-8B on a shared x and
    all seven linears on four inputs (salient columns on o, bias on down),
    each member against the oracle and against its single-linear call; a
    batch of one is that call, bit for bit."""

    backend = HipPackedBackend()
    shapes = syn.llama3_8b_layer()
    states = [syn.synthetic_packed_layer(s, seed=syn.BASE_SEED + 90 + i, salient=5 if i == 3 else 0, bias=i == 6)
              for i, s in enumerate(shapes)]
    layers = [backend.prepare(st, "cuda") for st in states]
    xa, xo, xm = (syn.synthetic_activations(tokens, 4096, seed=s, device="cuda") for s in (1, 2, 3))
    xd = syn.synthetic_activations(tokens, 14336, seed=4, device="cuda")
    inputs = [xa, xa, xa, xo, xm, xm, xd]
    _say("prefill qkv batch", tokens)
    qkv = backend.linear_batch(inputs[:3], layers[:3])
    _say("prefill layer batch", tokens)
    whole = backend.linear_batch(inputs, layers)
    again = backend.linear_batch(inputs, layers)
    for i, (state, x) in enumerate(zip(states, inputs)):
        expected = orc.packed_forward(orc.operands_from_state(state), x.cpu())
        single = backend.linear(x, layers[i])
        for name, y in (("layer", whole[i]), ("qkv", qkv[i] if i < 3 else None)):
            if y is None:
                continue
            err = orc.relative_l2(y, expected)
            assert err <= REL_L2, (state.spec.name, name, tokens, err)
            assert orc.relative_l2(y, single) <= 1e-4, (state.spec.name, name, tokens)
        assert torch.equal(whole[i], again[i])
        (one,) = backend.linear_batch([x], [layers[i]])
        assert torch.equal(one, single), state.spec.name
    print(f"  M={tokens}: 7 members within {REL_L2} of the oracle", flush=True)


@pytest.mark.parametrize("tokens", [40, 129])
def test_prefill_batch_ragged_members(tokens):
    """Members of unlike geometry in one prefill batch: word tails, partial
    tiles, an input width that is not a multiple of 8 (the generic row pass for
    the whole batch), salient columns and bias, members whose K is split beside
    members whose K is not (empty reduction ranges), bf16 outputs."""

    backend = HipPackedBackend()
    geometries = [(35, 17, 33, 3), (200, 130, 129, 5), (1152, 864, 768, 0), (640, 257, 96, 31),
                  (4096, 1024, 655, 0)]
    states = [syn.synthetic_packed_layer(syn.LinearShape(f"blocks.0.m{i}", g[0], g[1], g[2]), seed=tokens + 7 * i,
                                         salient=g[3], bias=True) for i, g in enumerate(geometries)]
    layers = [backend.prepare(st, "cuda") for st in states]
    xs = [syn.synthetic_activations(tokens, g[0], seed=tokens + i, device="cuda") for i, g in enumerate(geometries)]
    _say("prefill ragged batch", tokens)
    ys = backend.linear_batch(xs, layers)
    outs = [torch.empty(tokens, g[1], dtype=torch.bfloat16, device="cuda") for g in geometries]
    backend.linear_batch(xs, layers, output_dtype=torch.bfloat16, outs=outs)
    for state, x, y, out in zip(states, xs, ys, outs):
        err = orc.relative_l2(y, orc.packed_forward(orc.operands_from_state(state), x.cpu()))
        assert err <= REL_L2, (state.spec.name, tokens, err)
        torch.testing.assert_close(out, y.to(torch.bfloat16), rtol=0, atol=0)
    # The vector row pass where every member allows it (widths divisible by 8).
    _say("prefill vector-row batch", tokens)
    ys = backend.linear_batch(xs[2:], layers[2:])
    for state, x, y in zip(states[2:], xs[2:], ys):
        err = orc.relative_l2(y, orc.packed_forward(orc.operands_from_state(state), x.cpu()))
        assert err <= REL_L2, (state.spec.name, tokens, err)


def test_prefill_batch_wide_blocks_at_2048():
    """Gate/up of Llama-3-8B at M = 2048: the batch takes the 128 x 256 block
    tile for its second GEMM (no member split) and matches the oracle."""

    backend = HipPackedBackend()
    shapes = syn.llama3_8b_layer()[4:6]
    states = [syn.synthetic_packed_layer(s, seed=syn.BASE_SEED + 95 + i) for i, s in enumerate(shapes)]
    layers = [backend.prepare(st, "cuda") for st in states]
    x = syn.synthetic_activations(2048, 4096, seed=9, device="cuda")
    _say("prefill gate/up batch", 2048)
    ys = backend.linear_batch([x, x], layers)
    for state, y, layer in zip(states, ys, layers):
        err = orc.relative_l2(y, orc.packed_forward(orc.operands_from_state(state), x.cpu()))
        assert err <= REL_L2, (state.spec.name, err)
        assert orc.relative_l2(y, backend.linear(x, layer)) <= 1e-4


@pytest.mark.parametrize("tokens", [1800, 2048])
def test_prefill_block_tile_does_not_change_results(tokens):
    """Gate/up of Llama-3-8B at M = 1800 and 2048: batched, the first GEMM
    runs as 128 x 256 blocks (300 / 320 of them); each linear alone runs it as
    128 x 128 blocks (the round model's choice at 150 / 160 wide blocks). Both
    tiles sum each output's K in the same order, so the batch equals each
    linear called on its own exactly, and both match the oracle."""

    backend = HipPackedBackend()
    shapes = syn.llama3_8b_layer()[4:6]
    states = [syn.synthetic_packed_layer(s, seed=syn.BASE_SEED + 93 + i) for i, s in enumerate(shapes)]
    layers = [backend.prepare(st, "cuda") for st in states]
    x = syn.synthetic_activations(tokens, 4096, seed=tokens, device="cuda")
    _say("prefill gate/up batch against single calls", tokens)
    ys = backend.linear_batch([x, x], layers)
    for state, y, layer in zip(states, ys, layers):
        assert torch.equal(y, backend.linear(x, layer)), state.spec.name
        err = orc.relative_l2(y, orc.packed_forward(orc.operands_from_state(state), x.cpu()))
        assert err <= REL_L2, (state.spec.name, err)
    assert all(torch.equal(a, b) for a, b in zip(ys, backend.linear_batch([x, x], layers)))


def test_prefill_wide_blocks_with_split_k_at_2048():
    """Down of Llama-3-8B at M = 2048 (K = 14336): its first GEMM splits K
    three ways and, by the round model, takes the 128 x 256 block tile, whose
    partial sums the split reduction adds in slice order."""

    backend = HipPackedBackend()
    shape = syn.llama3_8b_layer()[6]
    state = syn.synthetic_packed_layer(shape, seed=syn.BASE_SEED + 97)
    layer = backend.prepare(state, "cuda")
    x = syn.synthetic_activations(2048, shape.in_features, seed=10, device="cuda")
    _say("prefill down, split K, wide blocks", 2048)
    y = backend.linear(x, layer)
    err = orc.relative_l2(y, orc.packed_forward(orc.operands_from_state(state), x.cpu()))
    assert err <= REL_L2, err
    assert torch.equal(y, backend.linear(x, layer))


# --- exact properties at the benchmark sizes -------------------------------------------

_PROPERTY_CASES = [
    ("qwen3 gate decode", syn.qwen3_8b_layer()[4], 1),
    ("qwen3 down decode", syn.qwen3_8b_layer()[6], 1),
    ("qwen3 q decode", syn.qwen3_8b_layer()[0], 16),
    ("llama gate prefill", syn.llama3_8b_layer()[4], 64),
    ("llama down prefill, split K", syn.llama3_8b_layer()[6], 2048),
]


@pytest.mark.parametrize("case", _PROPERTY_CASES, ids=[c[0] for c in _PROPERTY_CASES])
def test_power_of_two_input_scaling_is_exact(case):
    """y(2^k x) == 2^k y(x) bit for bit on the tiled paths (no bias): decode
    takes one power of two per activation chunk and prefill one per token
    row, so scaling x by 2^k shifts those exponents and nothing else, and the
    fp32 output comes out scaled exactly."""

    name, shape, tokens = case
    backend = HipPackedBackend()
    layer = backend.prepare(syn.synthetic_packed_layer(shape, seed=syn.BASE_SEED + 101), "cuda")
    x = syn.synthetic_activations(tokens, shape.in_features, seed=11, device="cuda")
    _say("power-of-two scaling", name, tokens)
    y = backend.linear(x, layer)
    for k in (-3, 5):
        assert torch.equal(backend.linear(x * 2.0**k, layer), y * 2.0**k), (name, k)


@pytest.mark.parametrize("case", _PROPERTY_CASES, ids=[c[0] for c in _PROPERTY_CASES])
def test_one_sign_flip_in_u_moves_one_output_column(case):
    """Flipping sign bit (o, r) of U changes output column o alone: every
    other output stays bit-identical (column o' reads row o' of U only), and
    column o moves by the oracle's difference, -2 sgn(U[o, r]) s_out[o] lm[r]
    per token."""

    name, shape, tokens = case
    backend = HipPackedBackend()
    state = syn.synthetic_packed_layer(shape, seed=syn.BASE_SEED + 103)
    o, r = shape.out_features // 3, shape.rank - 2
    words = state.left_words.clone()
    words.numpy().view(np.uint32)[o, r // 32] ^= np.uint32(1 << (r % 32))
    flipped = replace(state, left_words=words)
    x = syn.synthetic_activations(tokens, shape.in_features, seed=13, device="cuda")
    _say("one sign flip in U", name, tokens, (o, r))
    y = backend.linear(x, backend.prepare(state, "cuda"))
    y2 = backend.linear(x, backend.prepare(flipped, "cuda"))
    others = torch.ones(shape.out_features, dtype=torch.bool, device=y.device)
    others[o] = False
    assert torch.equal(y[:, others], y2[:, others]), name
    got = (y2[:, o] - y[:, o]).cpu()
    expected = (orc.packed_forward(orc.operands_from_state(flipped), x.cpu())[:, o]
                - orc.packed_forward(orc.operands_from_state(state), x.cpu())[:, o])
    assert float(expected.abs().min()) > 0.0
    assert orc.relative_l2(got, expected) <= REL_L2, name


def test_batch_rejects_mixed_launch_structures():
    state = syn.synthetic_packed_layer(syn.qwen3_8b_layer()[1], seed=3)
    split, fused = HipPackedBackend(decode_launch="split"), HipPackedBackend(decode_launch="fused")
    a, b = split.prepare(state, "cuda"), fused.prepare(state, "cuda")
    x = syn.synthetic_activations(1, 4096, seed=1, device="cuda")
    with pytest.raises(_native.NativeCallError):
        split.linear_batch([x, x], [a, b])


def test_batch_rejects_duplicate_members():
    backend = HipPackedBackend()
    state = syn.synthetic_packed_layer(syn.qwen3_8b_layer()[1], seed=3)
    layer = backend.prepare(state, "cuda")
    x = syn.synthetic_activations(1, 4096, seed=1, device="cuda")
    with pytest.raises(ValueError, match="distinct"):
        backend.linear_batch([x, x], [layer, layer])


def test_read_stream_probe_reads_every_word():
    """nq_read_stream (the bench's HBM read ceiling) touches every word: the
    XOR of its per-workgroup sinks equals the XOR of the buffer."""

    g = torch.Generator().manual_seed(17)
    data = torch.randint(-(2**31), 2**31, (3_000_004,), generator=g, dtype=torch.int64).to(torch.int32)
    sink = torch.zeros(4096, dtype=torch.int32, device="cuda")
    lib = _native.load()
    dev = data.cuda()
    status = lib.nq_read_stream(dev.data_ptr(), dev.numel() * 4, sink.data_ptr(), sink.numel(),
                                _native.current_stream_handle(dev.device))
    assert status == _native.NQ_OK
    expected = np.bitwise_xor.reduce(data.numpy().view(np.uint32))
    assert np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32)) == expected
    assert lib.nq_read_stream(dev.data_ptr(), 20, sink.data_ptr(), 1, None) == _native.NQ_ERR_ALIGNMENT
