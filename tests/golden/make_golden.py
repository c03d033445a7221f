"""Write ``reference_fixtures.json``: the reference tests' fixtures evaluated exactly.

The packed linear has no stored golden vectors in the reference; its tests build
small fixtures from closed forms and compare implementations. This script
rebuilds those fixtures from their closed forms (transcribed from the reference
tests, cited per fixture) and evaluates the layer with exact rational
arithmetic (``fractions.Fraction`` over the exact float32 values), with its own
integer bit packing. Nothing here imports torch, numpy, the oracle or the
reference, so the fixtures pin the oracle independently.

Run: ``python tests/golden/make_golden.py`` (rewrites the JSON next to it).
"""

from __future__ import annotations

import json
import struct
from fractions import Fraction
from pathlib import Path

OUT = Path(__file__).with_name("reference_fixtures.json")


def f32(value: float) -> float:
    """Round a Python float to the nearest float32, returned as a Python float."""

    return struct.unpack("<f", struct.pack("<f", value))[0]


def exact(value: float) -> Fraction:
    return Fraction(f32(value))


def linspace32(start: float, stop: float, steps: int) -> list[float]:
    """torch.linspace values in float32 (start + i*step, step computed in float32,
    with the second half mirrored from the end as torch does)."""

    if steps == 1:
        return [f32(start)]
    step = f32((stop - start) / (steps - 1))
    half = steps // 2
    values = []
    for i in range(steps):
        if i < half:
            values.append(f32(start + step * i))
        else:
            values.append(f32(stop - step * (steps - 1 - i)))
    return values


def pack_row(signs: list[int]) -> list[int]:
    """Pure-integer packing: bit c%32 of word c//32 set when sign is -1; int32 view."""

    words = []
    for base in range(0, len(signs), 32):
        acc = 0
        for bit, sign in enumerate(signs[base : base + 32]):
            if sign < 0:
                acc |= 1 << bit
        words.append(acc - (1 << 32) if acc >= 1 << 31 else acc)
    return words


def forward(fixture: dict, x_rows: list[list[float]]) -> list[list[float]]:
    """Exact y for each token row: salient columns' scale_pre masked to zero
    (src/nanoquant/runtime/reference.py:101-106), int8 salient values times
    their scales (reference.py:93-98)."""

    left, right = fixture["left"], fixture["right"]
    pre = [exact(v) for v in fixture["scale_pre"]]
    for index in fixture.get("outlier_indices", []):
        pre[index] = Fraction(0)
    mid = [exact(v) for v in fixture["scale_mid"]]
    post = [exact(v) for v in fixture["scale_post"]]
    bias = [exact(v) for v in fixture.get("bias", [0.0] * len(post))]
    idx = fixture.get("outlier_indices", [])
    values = fixture.get("outlier_values", [])
    scales = fixture.get("outlier_scales")
    outputs = []
    for row in x_rows:
        x = [exact(v) for v in row]
        latent = [
            sum((x[i] * pre[i] * right[r][i] for i in range(len(x))), Fraction(0)) * mid[r]
            for r in range(len(mid))
        ]
        y = []
        for o in range(len(post)):
            acc = sum((left[o][r] * latent[r] for r in range(len(mid))), Fraction(0)) * post[o]
            for k, col in enumerate(idx):
                weight = Fraction(values[o][k])
                if scales is not None:
                    scale = scales[o][k] if isinstance(scales[0], list) else scales[k]
                    weight *= exact(scale)
                acc += x[col] * weight
            y.append(float(acc + bias[o]))
        outputs.append(y)
    return outputs


def fixture_backend_4x3() -> dict:
    """tests/unit/test_runtime_backend.py:43-71 (4->3, rank 2, int8 outlier, bias).
    Its scales are [out, 1] (legal in the logical state only) and scale_pre is
    non-zero at the salient column, so the reference's masking is exercised."""

    fixture = {
        "name": "backend_4x3_rank2_int8_outlier",
        "source": "tests/unit/test_runtime_backend.py:43-71",
        "in_features": 4,
        "out_features": 3,
        "rank": 2,
        "left": [[1, -1], [-1, 1], [1, 1]],
        "right": [[1, -1, 1, -1], [-1, -1, 1, 1]],
        "scale_pre": [0.75, 1.0, 1.25, 1.5],
        "scale_mid": [0.5, 1.5],
        "scale_post": [1.25, 0.75, 1.5],
        "bias": [0.1, -0.2, 0.3],
        "outlier_indices": [1],
        "outlier_values": [[2], [-1], [3]],
        "outlier_scales": [[0.25], [0.5], [0.125]],
        "x": [[0.25, -0.5, 1.0, 0.75], [-1.0, 0.5, 0.125, -0.25]],
    }
    return fixture


def fixture_packed_35x3() -> dict:
    """tests/unit/test_runtime_packed.py:71-106 (35->3, rank 33, salient {1, 34})."""

    left = [[1 if (o * 33 + r) % 2 == 0 else -1 for r in range(33)] for o in range(3)]
    right = [[-1 if (r * 35 + i) % 5 == 0 else 1 for i in range(35)] for r in range(33)]
    scale_pre = [0.5, 0.0, *linspace32(0.5, 1.5, 32), 0.0]
    fixture = {
        "name": "packed_35x3_rank33_int8_salient",
        "source": "tests/unit/test_runtime_packed.py:71-106",
        "in_features": 35,
        "out_features": 3,
        "rank": 33,
        "left": left,
        "right": right,
        "scale_pre": scale_pre,
        "scale_mid": linspace32(0.75, 1.25, 33),
        "scale_post": linspace32(1.0, 1.5, 3),
        "bias": [0.1, -0.2, 0.3],
        "outlier_indices": [1, 34],
        "outlier_values": [[1, -2], [3, -4], [5, -6]],
        "outlier_scales": [0.25, 0.5],
        # linspace(-1, 1, 70).reshape(2, 35), the CUDA tests' input
        # (tests/unit/test_runtime_cuda_backend.py:553).
        "x": [row for row in (lambda v: [v[:35], v[35:]])(linspace32(-1.0, 1.0, 70))],
    }
    return fixture


def main() -> None:
    fixtures = [fixture_backend_4x3(), fixture_packed_35x3()]
    for fixture in fixtures:
        fixture["left_words"] = [pack_row(row) for row in fixture["left"]]
        fixture["right_words"] = [pack_row(row) for row in fixture["right"]]
        fixture["expected_y"] = forward(fixture, fixture["x"])
    known_words = {
        "source": "tests/unit/test_runtime_packed.py:42-50",
        "rows": [
            [-1 if c in (0, 1, 31) else 1 for c in range(32)],
            [-1] * 32,
        ],
        "words": [[-(2**31) + 3], [-1]],
    }
    assert [pack_row(r) for r in known_words["rows"]] == known_words["words"]
    payload = {
        "generator": "tests/golden/make_golden.py",
        "arithmetic": "exact rational over float32 inputs, rounded to float64",
        "known_answer_words": known_words,
        "fixtures": fixtures,
    }
    OUT.write_text(json.dumps(payload, indent=1) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
