"""Packed artifact format: write, open (manifest, sizes, hashes, headers), load a
layer, and the rejection cases of the reference's tests
(tests/unit/test_runtime_packed_artifact.py:25-200). CPU, plus one GPU test that
runs a loaded layer on the HIP backend against the oracle."""

from __future__ import annotations

import json
from pathlib import Path

import pytest
import torch

from conftest import gpu_available
from nanoquant_amd.runtime import PACKED_TENSOR_NAMESPACE, LogicalLayerState, QuantizedLinearSpec, pack_logical_layer
from nanoquant_amd.runtime.packed_artifact import (
    PackedArtifactError,
    RuntimeModelMetadata,
    open_packed_artifact,
    write_packed_artifact,
)


def _logical(name: str, *, outliers: bool) -> LogicalLayerState:
    """The reference test's 35 -> 3, rank 33 layer (tests/unit/test_runtime_packed_artifact.py:25-63)."""

    spec = QuantizedLinearSpec(
        name, "nanoquant-v1", 35, 3, 33, "float32", "float32",
        outlier_count=2 if outliers else 0, outlier_value_dtype="int8" if outliers else None,
        has_outlier_scales=outliers, has_bias=True,
    )
    return LogicalLayerState(
        spec,
        torch.where(torch.arange(99).reshape(3, 33) % 2 == 0, torch.ones(3, 33), -torch.ones(3, 33)),
        torch.where(torch.arange(33 * 35).reshape(33, 35) % 3 == 0, -torch.ones(33, 35), torch.ones(33, 35)),
        (torch.cat((torch.tensor([0.5, 0.0]), torch.linspace(0.5, 1.5, 32), torch.zeros(1)))
         if outliers else torch.linspace(0.5, 1.5, 35)),
        torch.linspace(0.75, 1.25, 33),
        torch.linspace(1.0, 1.5, 3),
        torch.tensor([0.1, -0.2, 0.3]),
        torch.tensor([1, 34], dtype=torch.int32) if outliers else None,
        torch.tensor([[1, -2], [3, -4], [5, -6]], dtype=torch.int8) if outliers else None,
        torch.tensor([0.25, 0.5]) if outliers else None,
    )


def _metadata() -> RuntimeModelMetadata:
    return RuntimeModelMetadata("fixture/model", "revision", "fixture", "config", "tokenizer")


def _write(tmp_path: Path):
    first = pack_logical_layer(_logical("blocks.0.linear", outliers=True))
    second = pack_logical_layer(_logical("blocks.1.linear", outliers=False))
    artifact = write_packed_artifact(tmp_path / "packed", _metadata(), "ab" * 32, {0: (first,), 1: (second,)})
    return artifact, first, second


def test_write_open_and_load_round_trip(tmp_path: Path):
    artifact, first, second = _write(tmp_path)
    m = artifact.manifest
    assert m.layout.version == "llama.cpp-i32-lsb-v1"
    assert m.layout.reference.commit == "da52148384591f4b0d87d58c12862e30f43014f1"
    assert m.layer_count == 2 and m.logical_descriptor_sha256 == "ab" * 32
    assert [b.path for b in m.blocks] == ["weights/block-00000.safetensors", "weights/block-00001.safetensors"]
    assert all(t.key.startswith(f"{PACKED_TENSOR_NAMESPACE}.") for b in m.blocks for l in b.layers for t in l.tensors)
    assert artifact.layer_names() == ["blocks.0.linear", "blocks.1.linear"]
    loaded = artifact.load_layer("blocks.0.linear")
    assert loaded.spec == first.spec
    for role in ("left_words", "right_words", "scale_pre", "scale_mid", "scale_post", "bias",
                 "outlier_indices", "outlier_values", "outlier_scales"):
        assert torch.equal(getattr(loaded, role), getattr(first, role)), role
    restored = loaded.to_logical()
    source = _logical("blocks.0.linear", outliers=True)
    assert torch.equal(restored.left_binary, source.left_binary)
    assert torch.equal(restored.right_binary, source.right_binary)
    assert artifact.load_layer("blocks.1.linear").spec == second.spec
    # the manifest is plain sorted JSON of the dataclasses
    payload = json.loads((artifact.root / "nanoquant-packed-model.json").read_text())
    assert payload["artifact_format"] == "nanoquant-packed-model" and payload["schema_version"] == 1
    assert payload["blocks"][0]["layers"][0]["spec"]["name"] == "blocks.0.linear"
    with pytest.raises(KeyError):
        artifact.load_layer("blocks.2.linear")


def test_open_does_not_load_payloads(tmp_path: Path):
    artifact, first, _ = _write(tmp_path)
    (artifact.root / artifact.manifest.blocks[1].path).unlink()
    assert torch.equal(artifact.load_layer(first.spec.name).left_words, first.left_words)


def test_rejects_corrupt_shard(tmp_path: Path):
    artifact, _, _ = _write(tmp_path)
    shard = artifact.root / artifact.manifest.blocks[0].path
    with shard.open("r+b") as stream:
        stream.seek(-1, 2)
        last = stream.read(1)
        stream.seek(-1, 2)
        stream.write(bytes([last[0] ^ 0xFF]))
    with pytest.raises(PackedArtifactError, match="shard hash differs"):
        open_packed_artifact(artifact.root)


def _edit_descriptor(root: Path, edit) -> None:
    path = root / "nanoquant-packed-model.json"
    payload = json.loads(path.read_text())
    edit(payload)
    path.write_text(json.dumps(payload))


def test_rejects_future_schema(tmp_path: Path):
    artifact, _, _ = _write(tmp_path)
    _edit_descriptor(artifact.root, lambda p: p.__setitem__("schema_version", 2))
    with pytest.raises(PackedArtifactError, match="unsupported packed artifact schema"):
        open_packed_artifact(artifact.root)


def test_rejects_noncanonical_tensor_key(tmp_path: Path):
    artifact, _, _ = _write(tmp_path)
    _edit_descriptor(artifact.root,
                     lambda p: p["blocks"][0]["layers"][0]["tensors"][0].__setitem__("key", "factor_left_words"))
    with pytest.raises(PackedArtifactError, match="tensor key differs"):
        open_packed_artifact(artifact.root, verify_hashes=False)


def test_rejects_unknown_field_and_escaping_path(tmp_path: Path):
    artifact, _, _ = _write(tmp_path)
    _edit_descriptor(artifact.root, lambda p: p.__setitem__("extra", 1))
    with pytest.raises(PackedArtifactError, match="unknown fields"):
        open_packed_artifact(artifact.root)
    _edit_descriptor(artifact.root, lambda p: (p.pop("extra"), p["blocks"][0].__setitem__("path", "../x.safetensors")))
    with pytest.raises(PackedArtifactError, match="not canonical"):
        open_packed_artifact(artifact.root)


def test_refuses_overwrite_and_leaves_no_staging(tmp_path: Path):
    artifact, first, _ = _write(tmp_path)
    with pytest.raises(FileExistsError, match="already exists"):
        write_packed_artifact(artifact.root, _metadata(), "ab" * 32, {0: (first,)})
    with pytest.raises(ValueError, match="contiguous"):
        write_packed_artifact(tmp_path / "gap", _metadata(), "ab" * 32, {1: (first,)})
    assert not list(tmp_path.glob(".nanoquant-packed-*"))


def _small_decoder():
    from nanoquant_amd import synthetic as syn
    from nanoquant_amd.runtime.decoder_shell import DecoderShellConfig

    config = DecoderShellConfig(layers=2, hidden=256, intermediate=768, q_heads=4, kv_heads=2, head_dim=64, vocab=500)
    return config, syn.synthetic_decoder(config, seed=syn.BASE_SEED + 71, random_norms=True)


def test_decoder_weights_from_artifact(tmp_path: Path):
    from nanoquant_amd.runtime.decoder_shell import dense_tensors, load_decoder_weights

    config, weights = _small_decoder()
    blocks = {i: list(layer.linears.values()) for i, layer in enumerate(weights.layers)}
    artifact = write_packed_artifact(tmp_path / "decoder", _metadata(), "ef" * 32, blocks)
    loaded = load_decoder_weights(artifact, dense_tensors(weights), config)
    assert torch.equal(loaded.embed, weights.embed) and torch.equal(loaded.final_norm, weights.final_norm)
    for got, want in zip(loaded.layers, weights.layers):
        assert torch.equal(got.q_norm, want.q_norm) and torch.equal(got.post_norm, want.post_norm)
        for role, state in want.linears.items():
            assert got.linears[role].spec == state.spec
            assert torch.equal(got.linears[role].left_words, state.left_words)


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a HIP device")
def test_decoder_from_artifact_generates_like_in_memory(tmp_path: Path):
    from nanoquant_amd.runtime.decoder_shell import PackedDecoder, dense_tensors, load_decoder_weights

    config, weights = _small_decoder()
    blocks = {i: list(layer.linears.values()) for i, layer in enumerate(weights.layers)}
    artifact = write_packed_artifact(tmp_path / "decoder", _metadata(), "ef" * 32, blocks)
    device = torch.device("cuda", 0)
    prompt = torch.randint(0, config.vocab, (30,), generator=torch.Generator().manual_seed(9)).to(device)
    direct = PackedDecoder(config, weights, device=device, max_positions=64).generate_greedy(prompt, 12)
    loaded = load_decoder_weights(artifact, dense_tensors(weights), config, device=device)
    via_artifact = PackedDecoder(config, loaded, device=device, max_positions=64).generate_greedy(prompt, 12)
    assert torch.equal(direct, via_artifact)


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a HIP device")
def test_loaded_layer_runs_on_hip_backend(tmp_path: Path):
    from nanoquant_amd import synthetic as syn
    from nanoquant_amd.runtime import HipPackedBackend
    from oracle import nq_oracle as orc

    shapes = syn.qwen3_8b_layer(0)
    states = [syn.synthetic_packed_layer(s, seed=syn.BASE_SEED + 70 + i) for i, s in enumerate(shapes[:2])]
    artifact = write_packed_artifact(tmp_path / "qwen", _metadata(), "cd" * 32, {0: states})
    device = torch.device("cuda", 0)
    backend = HipPackedBackend()
    for state in states:
        layer = backend.prepare(artifact.load_layer(state.spec.name, device), device)
        x = syn.synthetic_activations(4, state.spec.in_features, seed=3)
        y = backend.linear(x.to(device), layer)
        assert orc.relative_l2(y, orc.packed_forward(orc.operands_from_state(state), x)) <= 2e-3


# --- an artifact written by the reference's own writer --------------------------------
#
# tests/golden/reference_artifact/ was written by the reference's
# write_packed_artifact and pack_logical_layer (tests/golden/make_artifact_fixture.py)
# from the dense layers of tests/golden/artifact_recipe.py.

GOLDEN = Path(__file__).resolve().parent / "golden"
REFERENCE_ARTIFACT = GOLDEN / "reference_artifact"


def _recipe_states():
    import sys

    sys.path.insert(0, str(GOLDEN))
    from artifact_recipe import LAYERS, dense_layer

    states = []
    for i in range(len(LAYERS)):
        kwargs = dense_layer(i)
        spec = QuantizedLinearSpec(**kwargs.pop("spec_args"))
        states.append(pack_logical_layer(LogicalLayerState(spec, **kwargs)))
    return states


_ROLES = ("left_words", "right_words", "scale_pre", "scale_mid", "scale_post", "bias", "outlier_indices",
          "outlier_values", "outlier_scales", "patch_left", "patch_right")


def test_reference_written_artifact_opens_and_loads_exactly():
    """The loader accepts the reference writer's manifest and shards (strict
    field check, sizes, SHA-256, tensor headers) and each loaded layer equals
    this package's packing of the same dense layer: words bit for bit,
    scales and sidecars value for value, same spec."""

    artifact = open_packed_artifact(REFERENCE_ARTIFACT)
    manifest = json.loads((REFERENCE_ARTIFACT / "nanoquant-packed-model.json").read_text())
    assert manifest["layer_count"] == 3 and len(manifest["blocks"]) == 2
    for expected in _recipe_states():
        loaded = artifact.load_layer(expected.spec.name)
        assert loaded.spec == expected.spec
        for role in _ROLES:
            a, b = getattr(loaded, role), getattr(expected, role)
            assert (a is None) == (b is None), role
            if a is not None:
                assert a.dtype == b.dtype and torch.equal(a, b), (expected.spec.name, role)


def test_reference_written_artifact_rejects_a_flipped_shard_byte(tmp_path: Path):
    import shutil

    copy = tmp_path / "artifact"
    shutil.copytree(REFERENCE_ARTIFACT, copy)
    shard = copy / "weights" / "block-00001.safetensors"
    data = bytearray(shard.read_bytes())
    data[-1] ^= 1
    shard.write_bytes(bytes(data))
    with pytest.raises(PackedArtifactError, match="hash"):
        open_packed_artifact(copy)


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a HIP device")
@pytest.mark.parametrize("tokens", [1, 5, 40])
def test_reference_written_artifact_runs_on_hip_backend(tokens):
    """Every layer of the reference-written artifact, loaded to the device and
    run on the HIP backend (decode and prefill token counts), against the oracle."""

    from nanoquant_amd.runtime import HipPackedBackend
    from oracle import nq_oracle as orc

    artifact = open_packed_artifact(REFERENCE_ARTIFACT)
    device = torch.device("cuda", 0)
    for backend in (HipPackedBackend(), HipPackedBackend(tiled_decode=False)):
        for i, name in enumerate(layer.spec.name for block in artifact.manifest.blocks for layer in block.layers):
            state = artifact.load_layer(name, device)
            layer = backend.prepare(state, device)
            g = torch.Generator().manual_seed(tokens * 10 + i)
            x = torch.randn(tokens, state.spec.in_features, generator=g).to(torch.bfloat16)
            y = backend.linear(x.to(device), layer)
            expected = orc.packed_forward(orc.operands_from_state(artifact.load_layer(name)), x)
            err = orc.relative_l2(y, expected)
            print(f"  {name} M={tokens} tiled={backend._tiled_decode} rel_l2={err:.2e}", flush=True)
            assert err <= 2e-3, (name, tokens, err)
