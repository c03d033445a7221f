"""bench.py's command line without a GPU: more than one GPU is refused with
exit status 2 and a message, before anything touches a device."""

from __future__ import annotations

import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused(capsys, monkeypatch):
    monkeypatch.delenv("WORLD_SIZE", raising=False)
    assert bench.main(["--gpus", "2"]) == 2
    assert "one GPU only" in capsys.readouterr().err


def test_a_distributed_launch_is_refused(capsys, monkeypatch):
    monkeypatch.setenv("WORLD_SIZE", "2")
    assert bench.main([]) == 2
    assert "WORLD_SIZE 2" in capsys.readouterr().err


def test_validation_reconstruction_matches_the_oracle():
    # The headline run's validation rebuilds each packed linear as a dense fp64
    # matrix from its words with torch bit operations; it must be the oracle's
    # dense reconstruction of the same layer.
    import torch

    from nanoquant_amd import synthetic as syn
    from oracle.nq_oracle import dense_forward, operands_from_state

    state = syn.synthetic_packed_layer(syn.LinearShape("v", 96, 40, 33), seed=syn.BASE_SEED + 90)
    w = bench._dense_weight64(state, "cpu")
    op = operands_from_state(state)
    expected = dense_forward(op, torch.eye(op.in_features, dtype=torch.float64)).T
    assert w.shape == (40, 96)
    assert torch.allclose(w, expected, rtol=1e-12, atol=0.0)


def test_validation_reference_model_matches_the_oracle_decoder():
    # The transformers model the validation builds, with the reconstructed
    # weights, must give the oracle decoder's logits on a small geometry.
    import pytest
    import torch

    pytest.importorskip("transformers")
    from nanoquant_amd import synthetic as syn
    from nanoquant_amd.runtime.decoder_shell import DecoderShellConfig
    from oracle import decoder_shell as ods
    from oracle.nq_oracle import operands_from_state, relative_l2

    config = DecoderShellConfig(layers=2, hidden=64, intermediate=160, q_heads=4, kv_heads=2, head_dim=32, vocab=97)
    weights = syn.synthetic_decoder(config, seed=syn.BASE_SEED + 91, random_norms=True)
    model = bench._transformers_qwen3(config, 64, "cpu")
    with torch.no_grad():
        model.model.embed_tokens.weight.copy_(weights.embed.float())
        model.lm_head.weight.copy_(weights.lm_head.float())
        model.model.norm.weight.copy_(weights.final_norm.float())
        for block, layer in zip(model.model.layers, weights.layers):
            block.input_layernorm.weight.copy_(layer.input_norm.float())
            block.post_attention_layernorm.weight.copy_(layer.post_norm.float())
            block.self_attn.q_norm.weight.copy_(layer.q_norm.float())
            block.self_attn.k_norm.weight.copy_(layer.k_norm.float())
            for role, state in layer.linears.items():
                parent = block.self_attn if role in ("q_proj", "k_proj", "v_proj", "o_proj") else block.mlp
                getattr(parent, role).weight.copy_(bench._dense_weight64(state, "cpu").float())
        ids = torch.tensor([5, 17, 3, 88, 41, 0, 63, 29, 70, 12])
        got = model(input_ids=ids[None], use_cache=False).logits[0]
    geometry = ods.ShellGeometry(config.layers, config.hidden, config.intermediate, config.q_heads, config.kv_heads,
                                 config.head_dim, config.vocab, config.eps, config.rope_theta)
    ow = ods.ShellWeights(weights.embed, weights.lm_head, weights.final_norm,
                          [ods.LayerWeights(l.input_norm, l.post_norm, l.q_norm, l.k_norm,
                                            {r: operands_from_state(s) for r, s in l.linears.items()})
                           for l in weights.layers])
    oracle = ods.OracleDecoder(geometry, ow, max_positions=64)
    expected = oracle.forward(ids, 0)
    assert relative_l2(got, expected) < 1e-5
