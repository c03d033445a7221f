"""Dense inputs of the layers in the reference-written artifact fixture.

Pure torch, seeded, so ``make_artifact_fixture.py`` (which packs these layers
with the reference's packer and writes them with the reference's artifact
writer) and the tests (which pack them with this package's packer) build the
same tensors. Each entry: name, in, out, rank, scale dtype and the optional
sidecars; the geometries cover a word tail in both factors, int8 salient
columns with scales, bf16 salient values, a float patch and biases.
"""

from __future__ import annotations

import torch

LAYERS = (
    # name, in, out, rank, scale dtype, salient indices, salient dtype, bias, patch rank
    ("blocks.0.self_attn.k_proj", 35, 3, 33, torch.float16, (1, 34), torch.int8, True, 0),
    ("blocks.1.mlp.down_proj", 512, 128, 102, torch.float16, (), None, False, 0),
    ("blocks.1.mlp.up_proj", 96, 64, 40, torch.bfloat16, (0, 50, 95), torch.bfloat16, True, 3),
)
SEED = 20260715


def dense_layer(index: int) -> dict:
    """The tensors of layer `index` as keyword arguments of a logical layer
    state (plus ``spec_args`` for its QuantizedLinearSpec)."""

    name, n_in, n_out, rank, sdt, salient, odt, bias, patch = LAYERS[index]
    g = torch.Generator().manual_seed(SEED + index)
    signs = lambda r, c: torch.where(torch.rand(r, c, generator=g) < 0.5, -1.0, 1.0)  # noqa: E731
    scale = lambda n: torch.exp(0.25 * torch.randn(n, generator=g)).to(sdt)  # noqa: E731
    out = {
        "left_binary": signs(n_out, rank),
        "right_binary": signs(rank, n_in),
        "scale_pre": scale(n_in),
        "scale_mid": scale(rank),
        "scale_post": scale(n_out),
    }
    spec = {"name": name, "logical_format": "nanoquant-v1", "in_features": n_in, "out_features": n_out,
            "rank": rank, "factor_dtype": "float32", "scale_dtype": str(sdt).removeprefix("torch.")}
    if salient:
        idx = torch.tensor(salient, dtype=torch.int32)
        out["scale_pre"][idx.long()] = 0
        out["outlier_indices"] = idx
        if odt == torch.int8:
            out["outlier_values"] = torch.randint(-127, 128, (n_out, len(salient)), generator=g, dtype=torch.int8)
            out["outlier_scales"] = scale(len(salient))
        else:
            out["outlier_values"] = torch.randn(n_out, len(salient), generator=g).to(odt)
        spec.update(outlier_count=len(salient), outlier_value_dtype=str(odt).removeprefix("torch."),
                    has_outlier_scales=odt == torch.int8)
    if bias:
        out["bias"] = torch.randn(n_out, generator=g).to(sdt)
        spec.update(has_bias=True)
    if patch:
        out["patch_left"] = 0.1 * torch.randn(n_out, patch, generator=g)
        out["patch_right"] = 0.1 * torch.randn(patch, n_in, generator=g)
        spec.update(patch_rank=patch, patch_value_dtype="float32")
    out["spec_args"] = spec
    return out


# Block of each layer in the artifact.
BLOCKS = {0: (0,), 1: (1, 2)}
