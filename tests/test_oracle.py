"""Pin the CPU oracle: golden vectors from the reference tests' fixtures (exact
rational evaluation), known-answer words, the C restatement, the dense
reconstruction and closed forms. Planted mistakes live in the oracle here, on
the CPU, to show each check can fail."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import c_oracle
from oracle import nq_oracle as orc

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_fixtures.json").read_text())


def _fixture_operands(f: dict) -> orc.PackedOperands:
    scales = f.get("outlier_scales")
    return orc.PackedOperands(
        f["in_features"],
        f["out_features"],
        f["rank"],
        np.array(f["left_words"], dtype=np.int32),
        np.array(f["right_words"], dtype=np.int32),
        torch.tensor(f["scale_pre"], dtype=torch.float32),
        torch.tensor(f["scale_mid"], dtype=torch.float32),
        torch.tensor(f["scale_post"], dtype=torch.float32),
        torch.tensor(f["bias"], dtype=torch.float32) if "bias" in f else None,
        torch.tensor(f["outlier_indices"], dtype=torch.int32) if "outlier_indices" in f else None,
        torch.tensor(f["outlier_values"], dtype=torch.int8) if "outlier_values" in f else None,
        None if scales is None else torch.tensor(scales, dtype=torch.float32),
    )


# --- sign words -----------------------------------------------------------------


def test_known_answer_words():
    kaw = GOLDEN["known_answer_words"]
    rows = np.array(kaw["rows"], dtype=np.int8)
    expected = np.array(kaw["words"], dtype=np.int32)
    assert np.array_equal(orc.pack_signs(rows), expected)
    assert np.array_equal(c_oracle.pack(rows), expected)
    assert np.array_equal(orc.unpack_signs(expected, 2, 32), rows)
    assert np.array_equal(c_oracle.unpack(expected, 2, 32), rows)


@pytest.mark.parametrize("cols", (1, 31, 32, 33, 65, 128))
def test_round_trip_tail_widths(cols):
    # tests/unit/test_runtime_packed.py:27-39 pattern: every third entry negative.
    signs = np.where(np.arange(3 * cols).reshape(3, cols) % 3 == 0, -1, 1).astype(np.int8)
    words = orc.pack_signs(signs)
    assert words.dtype == np.int32 and words.shape == (3, orc.word_count(cols))
    assert np.array_equal(orc.unpack_signs(words, 3, cols), signs)
    assert np.array_equal(c_oracle.pack(signs), words)
    assert np.array_equal(c_oracle.unpack(words, 3, cols), signs)


def test_golden_fixture_words_match_both_packers():
    for f in GOLDEN["fixtures"]:
        for signs, words in ((f["left"], f["left_words"]), (f["right"], f["right_words"])):
            s = np.array(signs, dtype=np.int8)
            w = np.array(words, dtype=np.int32)
            assert np.array_equal(orc.pack_signs(s), w)
            assert np.array_equal(c_oracle.pack(s), w)


def test_padding_rejected():
    words = orc.pack_signs(np.ones((1, 33), dtype=np.int8))
    words[0, -1] = 2
    with pytest.raises(ValueError, match="non-zero padding bit"):
        orc.unpack_signs(words, 1, 33)
    with pytest.raises(ValueError, match="non-zero padding bit"):
        c_oracle.unpack(words, 1, 33)


def test_random_words_bit_exact_between_numpy_and_c():
    rng = np.random.default_rng(5)
    for rows, cols in ((7, 1), (5, 819), (3, 4096), (64, 35)):
        signs = np.where(rng.random((rows, cols)) < 0.5, -1, 1).astype(np.int8)
        words = orc.pack_signs(signs)
        assert np.array_equal(c_oracle.pack(signs), words)
        assert np.array_equal(c_oracle.unpack(words, rows, cols), signs)
        assert np.array_equal(orc.unpack_signs(words, rows, cols), signs)


# --- linear ----------------------------------------------------------------------


@pytest.mark.parametrize("index", range(len(GOLDEN["fixtures"])))
def test_oracle_matches_exact_golden_outputs(index):
    f = GOLDEN["fixtures"][index]
    op = _fixture_operands(f)
    x = torch.tensor(f["x"], dtype=torch.float32)
    expected = torch.tensor(f["expected_y"], dtype=torch.float64)
    torch.testing.assert_close(orc.packed_forward(op, x, dtype=torch.float64), expected, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(orc.packed_forward(op, x).double(), expected, rtol=2e-6, atol=2e-6)
    torch.testing.assert_close(orc.dense_forward(op, x), expected, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("index", range(len(GOLDEN["fixtures"])))
def test_c_oracle_matches_exact_golden_outputs(index):
    f = GOLDEN["fixtures"][index]
    op = _fixture_operands(f)
    sal = op.outlier_values.float() * op.outlier_scales.float()
    y = c_oracle.linear_f64(
        op.in_features, op.out_features, op.rank, op.left_words, op.right_words,
        op.scale_pre.numpy(), op.scale_mid.numpy(), op.scale_post.numpy(),
        np.array(f["x"], dtype=np.float32), bias=op.bias.numpy(),
        idx=op.outlier_indices.numpy(), sal=sal.numpy(),
    )
    np.testing.assert_allclose(y, np.array(f["expected_y"]), rtol=1e-12, atol=1e-12)


def _planted(op: orc.PackedOperands, x: torch.Tensor, mistake: str) -> torch.Tensor:
    """The oracle with one plausible mistake planted (CPU only)."""

    u = torch.from_numpy(orc.unpack_signs(op.left_words, op.out_features, op.rank)).double()
    v = torch.from_numpy(orc.unpack_signs(op.right_words, op.rank, op.in_features)).double()
    pre = op.scale_pre.double().clone()
    if mistake != "no_mask":
        pre[op.outlier_indices.long()] = 0
    mid, post = op.scale_mid.double(), op.scale_post.double()
    if mistake == "drop_mid":
        mid = torch.ones_like(mid)
    if mistake == "flip_sign":
        v = -v
    if mistake == "bit_order":
        v = torch.flip(v, dims=[1])
    xs = x.double()
    y = ((xs * pre) @ v.T * mid) @ (u * post[:, None]).T
    sal = op.outlier_values.double() * op.outlier_scales.double()
    if mistake != "drop_salient":
        y = y + xs[:, op.outlier_indices.long()] @ sal.T
    if mistake != "drop_bias":
        y = y + op.bias.double()
    return y


@pytest.mark.parametrize(
    "mistake", ["drop_mid", "flip_sign", "bit_order", "drop_salient", "drop_bias", "no_mask"]
)
def test_golden_checks_catch_planted_mistakes(mistake):
    caught = False
    for f in GOLDEN["fixtures"]:
        op = _fixture_operands(f)
        x = torch.tensor(f["x"], dtype=torch.float32)
        expected = torch.tensor(f["expected_y"], dtype=torch.float64)
        assert torch.allclose(_planted(op, x, "none"), expected, rtol=1e-12, atol=1e-12)
        if not torch.allclose(_planted(op, x, mistake), expected, rtol=1e-6, atol=1e-6):
            caught = True
    assert caught, mistake


def _random_operands(in_f, out_f, rank, seed, *, salient=0) -> orc.PackedOperands:
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    u = np.where(rng.random((out_f, rank)) < 0.5, -1, 1).astype(np.int8)
    v = np.where(rng.random((rank, in_f)) < 0.5, -1, 1).astype(np.int8)
    pre = torch.exp(0.25 * torch.randn(in_f, generator=g))
    idx = vals = scales = None
    if salient:
        idx = torch.sort(torch.randperm(in_f, generator=g)[:salient]).values.to(torch.int32)
        pre[idx.long()] = 0
        vals = torch.randint(-127, 128, (out_f, salient), generator=g).to(torch.int8)
        scales = torch.rand(salient, generator=g) / 64
    return orc.PackedOperands(
        in_f, out_f, rank, orc.pack_signs(u), orc.pack_signs(v), pre,
        torch.exp(0.25 * torch.randn(rank, generator=g)),
        torch.exp(0.25 * torch.randn(out_f, generator=g)),
        torch.randn(out_f, generator=g), idx, vals, scales,
    )


@pytest.mark.parametrize("shape", [(35, 17, 33), (64, 48, 32), (96, 64, 64), (1152, 96, 77)])
def test_oracle_agrees_with_c_restatement_and_dense_form(shape):
    in_f, out_f, rank = shape
    op = _random_operands(in_f, out_f, rank, seed=sum(shape), salient=3)
    x = torch.randn(4, in_f, generator=torch.Generator().manual_seed(1))
    torch_y = orc.packed_forward(op, x, dtype=torch.float64)
    sal = (op.outlier_values.float() * op.outlier_scales.float()).numpy()
    c_y = c_oracle.linear_f64(
        in_f, out_f, rank, op.left_words, op.right_words, op.scale_pre.numpy(),
        op.scale_mid.numpy(), op.scale_post.numpy(), x.numpy(), bias=op.bias.numpy(),
        idx=op.outlier_indices.numpy(), sal=sal,
    )
    np.testing.assert_allclose(torch_y.numpy(), c_y, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(orc.dense_forward(op, x), torch_y, rtol=1e-10, atol=1e-10)
    assert orc.relative_l2(orc.packed_forward(op, x), torch_y) < 1e-6


def test_closed_form_all_positive_unit_scales():
    # U = V = +1, unit scales: y_o = rank * sum_i x_i for every output.
    in_f, out_f, rank = 70, 9, 40
    op = orc.PackedOperands(
        in_f, out_f, rank,
        orc.pack_signs(np.ones((out_f, rank), dtype=np.int8)),
        orc.pack_signs(np.ones((rank, in_f), dtype=np.int8)),
        torch.ones(in_f), torch.ones(rank), torch.ones(out_f),
    )
    x = torch.randn(3, in_f, dtype=torch.float64)
    expected = (rank * x.sum(dim=1, keepdim=True)).expand(3, out_f)
    torch.testing.assert_close(orc.packed_forward(op, x, dtype=torch.float64), expected)


def test_single_bit_flip_changes_one_output_by_closed_form():
    op = _random_operands(40, 6, 33, seed=11)
    x = torch.randn(1, 40, dtype=torch.float64, generator=torch.Generator().manual_seed(2))
    base = orc.packed_forward(op, x, dtype=torch.float64)
    # Flip U[o, r]: y_o changes by -2 * sgn_old * s_out[o] * lm[r].
    o, r = 4, 32
    flipped = op.left_words.copy()
    flipped.view(np.uint32)[o, r // 32] ^= np.uint32(1 << (r % 32))
    op2 = orc.PackedOperands(**{**op.__dict__, "left_words": flipped})
    changed = orc.packed_forward(op2, x, dtype=torch.float64)
    v = torch.from_numpy(orc.unpack_signs(op.right_words, 33, 40)).double()
    lm = ((x * op.scale_pre.double()) @ v.T)[0, r] * op.scale_mid.double()[r]
    old = float(orc.unpack_signs(op.left_words, 6, 33)[o, r])
    delta = changed - base
    assert torch.allclose(delta[0, o], torch.tensor(-2 * old * float(op.scale_post[o]) * float(lm), dtype=torch.float64))
    others = [i for i in range(6) if i != o]
    assert torch.allclose(delta[0, others], torch.zeros(5, dtype=torch.float64), atol=1e-12)


def test_linearity_in_x():
    op = _random_operands(64, 12, 20, seed=3)
    op.bias = None
    g = torch.Generator().manual_seed(4)
    a, b = torch.randn(2, 64, dtype=torch.float64, generator=g), torch.randn(2, 64, dtype=torch.float64, generator=g)
    f = lambda t: orc.packed_forward(op, t, dtype=torch.float64)  # noqa: E731
    torch.testing.assert_close(f(2.0 * a - 3.0 * b), 2.0 * f(a) - 3.0 * f(b))


def test_row_sidecar_patch_is_an_int8_gemv_into_selected_rows():
    out_f, in_f = 10, 50
    idx = torch.tensor([1, 4, 9], dtype=torch.int32)
    vals = torch.randint(-127, 128, (3, in_f), dtype=torch.int8, generator=torch.Generator().manual_seed(8))
    scales = torch.tensor([0.5, 0.25, 2.0])
    left, right = orc.row_sidecar_as_patch(out_f, idx, vals, scales)
    x = torch.randn(2, in_f, dtype=torch.float64)
    via_patch = (x @ right.double().T) @ left.double().T
    direct = torch.zeros(2, out_f, dtype=torch.float64)
    direct.index_add_(1, idx.long(), (x @ vals.double().T) * scales.double())
    torch.testing.assert_close(via_patch, direct)
