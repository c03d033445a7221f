"""Compact right-factor codecs: the numpy oracle (oracle/codecs.py) against the
reference tests' known answers and brute force, the runtime's host conversion
against the oracle, and (GPU) the device expansion used by
``HipPackedBackend.prepare`` against both."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import gpu_available
from nanoquant_amd.runtime import PackedLayerState, QuantizedLinearSpec, pack_sign_matrix
from nanoquant_amd.runtime import codecs as rc
from oracle import codecs as oc


def _rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


# --------------------------------------------------------------------- oracle pins
def test_stream_sizes_and_round_trip_match_reference_known_answers():
    # tests/unit/test_runtime_mixed_v.py:32-46
    indices = (np.arange(34).reshape(2, 17) * 29) % 1024
    pairs = (np.arange(34).reshape(2, 17) * 13) % 496
    payload = oc.pack_records(indices | (pairs << 10), 19)
    assert payload.size == 21 == oc.payload_words(34, 19)
    assert oc.payload_words(1088 * 216, 19) == 139_536
    back = oc.unpack_records(payload, 34, 19)
    assert np.array_equal(back & 1023, indices.reshape(-1)) and np.array_equal(back >> 10, pairs.reshape(-1))
    # tests/unit/test_runtime_product_codebook.py:62-73
    idx = (np.arange(15).reshape(3, 5) * 7919) % 65536
    payload16 = oc.pack_records(idx, 16)
    assert payload16.shape == (8,)
    assert np.array_equal(oc.unpack_records(payload16, 15, 16), idx.reshape(-1))


@pytest.mark.parametrize("bits", [16, 19, 7, 32])
def test_record_stream_against_a_bit_list(bits):
    values = _rng(bits).integers(0, 1 << bits, size=37, dtype=np.uint64)
    stream = [(int(v) >> j) & 1 for v in values for j in range(bits)]
    stream += [0] * (-len(stream) % 32)
    expected = [sum(stream[32 * w + j] << j for j in range(32)) for w in range(len(stream) // 32)]
    assert oc.pack_records(values, bits).view(np.uint32).tolist() == expected


def test_pair_ids_are_the_lexicographic_bit_pairs():
    pairs = [(a, b) for a in range(32) for b in range(a + 1, 32)]
    assert len(pairs) == oc.MIXED_V_PAIRS == rc.MIXED_V_CORRECTION_PAIR_COUNT
    assert [oc.pair_bits(i) for i in range(len(pairs))] == pairs
    table = rc.mixed_v_correction_pair_table()
    assert [(int(t) & 0xFF, int(t) >> 8) for t in table[:496]] == pairs and not table[496:].any()


def test_transpose_oracle_is_the_sign_transpose():
    signs = torch.where(torch.from_numpy(_rng(3).integers(0, 2, (37, 45))) == 1, -1.0, 1.0)
    words = pack_sign_matrix(signs).numpy()
    assert np.array_equal(oc.transpose_signs(words, 37, 45), pack_sign_matrix(signs.T.contiguous()).numpy())


# --------------------------------------------------------------------- runtime (host)
def _mixed_fixture():
    """tests/unit/test_runtime_mixed_v.py:49-118: codebook[0] = 0x12345678, codebook[1] = 3,
    records (0, pair 0) and (1, pair 0); pair 0 flips bits 0 and 1."""

    spec = QuantizedLinearSpec("blocks.0.linear", "nanoquant-v1", 35, 3, 7, "float32", "float32")
    codebook = torch.zeros(1024, dtype=torch.int32)
    codebook[0], codebook[1] = 0x12345678, 3
    indices = torch.tensor([[0, 1]] * 5, dtype=torch.int32)
    pairs = torch.zeros_like(indices)
    free = pack_sign_matrix(torch.where(torch.arange(70).reshape(2, 35) % 3 == 0, -1.0, 1.0))
    left = pack_sign_matrix(torch.where(torch.arange(21).reshape(3, 7) % 2 != 0, 1.0, -1.0))
    scales = (torch.linspace(0.5, 1.5, 35), torch.linspace(0.75, 1.25, 7), torch.linspace(1.0, 1.5, 3))
    state = rc.MixedVLayerState(spec, rc.MIXED_V_FORMAT_VERSION, 2, left, free,
                                rc.pack_mixed_v_records(indices, pairs), codebook, *scales)
    return state, free


def test_mixed_v_fixture_decodes_to_the_reference_words():
    state, free = _mixed_fixture()
    expected = torch.cat((free, torch.tensor([[0x12345678 ^ 3, 0]] * 5, dtype=torch.int32)))
    assert torch.equal(state.to_packed().right_words, expected)
    words, bad = oc.decode_mixed_v(free.numpy(), state.coded_payload.numpy(), state.codebook_words.numpy(), 7, 2)
    assert bad == 0 and np.array_equal(words, expected.numpy())


def test_mixed_v_rejections():
    with pytest.raises(ValueError, match="496 valid pairs"):
        rc.unpack_mixed_v_records(torch.tensor([496 << 10], dtype=torch.int32), (1, 1))
    padded = rc.pack_mixed_v_records(torch.zeros((1, 1), dtype=torch.int32), torch.zeros((1, 1), dtype=torch.int32))
    padded[0] = -(1 << 31)
    with pytest.raises(ValueError, match="non-zero padding"):
        rc.unpack_mixed_v_records(padded, (1, 1))
    state, free = _mixed_fixture()
    indices, pairs = rc.unpack_mixed_v_records(state.coded_payload, (5, 2))
    pairs[:, 1] = 30  # pair (0, 31): sets a pad bit of the 35-column tail word
    with pytest.raises(ValueError, match="non-zero padding bit"):
        rc.MixedVLayerState(state.spec, state.format, 2, state.left_words, free,
                            rc.pack_mixed_v_records(indices, pairs), state.codebook_words, state.scale_pre,
                            state.scale_mid, state.scale_post)


def _random_mixed(rank: int, in_features: int, free_rows: int, seed: int):
    g = _rng(seed)
    wpr = (in_features + 31) // 32
    free = g.integers(-(2**31), 2**31, size=(free_rows, wpr), dtype=np.int64).astype(np.int32)
    if in_features % 32:
        free[:, -1] &= (1 << (in_features % 32)) - 1
    idx = g.integers(0, 1024, size=(rank - free_rows, wpr))
    pair = g.integers(0, 496, size=(rank - free_rows, wpr))
    book = g.integers(-(2**31), 2**31, size=1024, dtype=np.int64).astype(np.int32)
    return free, oc.pack_records(idx | (pair << 10), 19), book


def test_mixed_v_host_decode_matches_oracle():
    free, payload, book = _random_mixed(40, 100, 9, 5)
    got = rc.decode_mixed_v_right_words(torch.from_numpy(free), torch.from_numpy(payload), torch.from_numpy(book),
                                        rank=40, in_features=100)
    expected, bad = oc.decode_mixed_v(free, payload, book, 40, 4)
    assert bad == 0 and np.array_equal(got.numpy(), expected)


def _table(words: list[int]) -> torch.Tensor:
    t = torch.ones((256, 16))
    for i, w in enumerate(words):
        t[i] = (1 - 2 * ((torch.tensor(w) >> torch.arange(16)) & 1)).float()
    return t.contiguous()


def _product_fixture(transposed: bool):
    """tests/unit/test_runtime_product_codebook.py:76-113."""

    spec = QuantizedLinearSpec("blocks.0.linear", "nanoquant-v1", 35, 3, 7, "float32", "float32")
    f_out, f_in = (35, 3) if transposed else (3, 35)
    signs = lambda r, c, m: torch.where(torch.arange(r * c).reshape(r, c) % m == 0, -1.0, 1.0).contiguous()  # noqa: E731
    coded = [0x12345678, 0x00000005] if f_in > 32 else [0x00000005]
    row = torch.tensor([0 if i == 0 else i | (i << 8) for i in range(len(coded))], dtype=torch.int32)
    indices = row[None, :].repeat(5, 1)
    return rc.ProductCodebookLayerState(
        spec, rc.PRODUCT_CODEBOOK_FORMAT_VERSION, transposed, 2, pack_sign_matrix(signs(f_out, 7, 3)),
        pack_sign_matrix(signs(2, f_in, 2)), rc.pack_product_codebook_indices(indices),
        rc.pack_product_half_table(_table([w & 0xFFFF for w in coded])),
        rc.pack_product_half_table(_table([(w >> 16) & 0xFFFF for w in coded])),
        torch.linspace(0.5, 1.5, f_in), torch.linspace(0.75, 1.25, 7), torch.linspace(1.0, 1.5, f_out))


@pytest.mark.parametrize("transposed", [False, True])
def test_product_codebook_host_conversion_matches_oracle(transposed):
    state = _product_fixture(transposed)
    packed = state.to_packed()
    assert packed.left_words.shape == (3, 1) and packed.right_words.shape == (7, 2)
    f_right = oc.decode_product_codebook(state.factor_right_free_words.numpy(),
                                         state.factor_right_coded_payload.numpy(), state.first_half_words.numpy(),
                                         state.second_half_words.numpy(), 7, (state.factor_in_features + 31) // 32)
    if transposed:
        assert np.array_equal(packed.left_words.numpy(), oc.transpose_signs(f_right, 7, 3))
        assert np.array_equal(packed.right_words.numpy(), oc.transpose_signs(state.factor_left_words.numpy(), 35, 7))
    else:
        assert np.array_equal(packed.right_words.numpy(), f_right)
    assert state.compact_logical_bits() == (
        state.factor_left_words.numel() * 32 + state.factor_right_free_words.numel() * 32 + state.record_count * 16
        + 8192 + 16 + (state.factor_in_features + 7 + state.factor_out_features) * 16)


def test_product_codebook_rejects_padding_record():
    payload = rc.pack_product_codebook_indices(((torch.arange(15).reshape(3, 5) * 7919) % 65536).to(torch.int32))
    payload[-1] |= torch.tensor(1 << 16, dtype=torch.int32)
    with pytest.raises(ValueError, match="non-zero padding"):
        rc.unpack_product_codebook_indices(payload, (3, 5))


# --------------------------------------------------------------------- device expansion
@pytest.mark.parametrize("rank,in_features,free_rows", [(3072, 4096, 1000), (819, 4096, 300), (40, 35, 9)])
@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a HIP device")
def test_device_mixed_v_matches_oracle(rank, in_features, free_rows):
    from nanoquant_amd.runtime import _native

    dev = torch.device("cuda", 0)
    free, payload, book = _random_mixed(rank, in_features, free_rows, rank)
    # plant invalid pair ids in two records (ids 500 and 511)
    records = oc.unpack_records(payload, (rank - free_rows) * ((in_features + 31) // 32), 19)
    records[3] = (records[3] & 1023) | (500 << 10)
    records[-1] = (records[-1] & 1023) | (511 << 10)
    payload = oc.pack_records(records, 19)
    wpr = (in_features + 31) // 32
    out = torch.empty((rank, wpr), dtype=torch.int32, device=dev)
    bad = torch.full((1,), 77, dtype=torch.int32, device=dev)
    p, f, b = (torch.from_numpy(a).to(dev) for a in (payload, free, book))
    _native.check("nq_decode_mixed_v_words", _native.load().nq_decode_mixed_v_words(
        f.data_ptr(), free_rows, p.data_ptr(), p.numel(), b.data_ptr(), rank, in_features, out.data_ptr(),
        bad.data_ptr(), _native.current_stream_handle(dev)))
    expected, expected_bad = oc.decode_mixed_v(free, payload, book, rank, wpr)
    assert np.array_equal(out.cpu().numpy(), expected)
    assert int(bad) == expected_bad == 2


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a HIP device")
def test_device_product_codebook_and_transpose_match_oracle():
    from nanoquant_amd.runtime import _native

    dev = torch.device("cuda", 0)
    g = _rng(11)
    rank, cols, free_rows = 2549, 1000, 700
    wpr = (cols + 31) // 32
    free = g.integers(-(2**31), 2**31, size=(free_rows, wpr), dtype=np.int64).astype(np.int32)
    idx = g.integers(0, 65536, size=(rank - free_rows) * wpr)
    payload = oc.pack_records(idx, 16)
    first = g.integers(-(2**15), 2**15, size=256).astype(np.int16)
    second = g.integers(-(2**15), 2**15, size=256).astype(np.int16)
    out = torch.empty((rank, wpr), dtype=torch.int32, device=dev)
    args = [torch.from_numpy(a).to(dev) for a in (free, payload, first, second)]
    lib, stream = _native.load(), _native.current_stream_handle(dev)
    _native.check("nq_decode_product_codebook_words", lib.nq_decode_product_codebook_words(
        args[0].data_ptr(), free_rows, args[1].data_ptr(), args[1].numel(), args[2].data_ptr(), args[3].data_ptr(),
        rank, cols, out.data_ptr(), stream))
    assert np.array_equal(out.cpu().numpy(), oc.decode_product_codebook(free, payload, first, second, rank, wpr))
    words = torch.from_numpy(g.integers(-(2**31), 2**31, size=(77, 5), dtype=np.int64).astype(np.int32))
    words[:, -1] &= (1 << (150 % 32)) - 1
    transposed = rc.transpose_signs_on_device(words.to(dev), 77, 150)
    assert np.array_equal(transposed.cpu().numpy(), oc.transpose_signs(words.numpy(), 77, 150))


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a HIP device")
def test_backend_prepares_compact_layers_like_their_packed_form():
    from nanoquant_amd import synthetic as syn
    from nanoquant_amd.runtime import HipPackedBackend

    dev = torch.device("cuda", 0)
    backend = HipPackedBackend()
    base = syn.synthetic_packed_layer(syn.qwen3_8b_layer()[1], seed=syn.BASE_SEED + 80)  # k_proj, rank 819
    wpr = base.right_words.shape[1]
    free_rows = 300
    g = _rng(12)
    book = torch.from_numpy(g.integers(-(2**31), 2**31, size=1024, dtype=np.int64).astype(np.int32))
    idx = torch.from_numpy(g.integers(0, 1024, size=(819 - free_rows, wpr)).astype(np.int32))
    pair = torch.from_numpy(g.integers(0, 496, size=(819 - free_rows, wpr)).astype(np.int32))
    mixed = rc.MixedVLayerState(base.spec, rc.MIXED_V_FORMAT_VERSION, free_rows, base.left_words,
                                base.right_words[:free_rows].contiguous(), rc.pack_mixed_v_records(idx, pair), book,
                                base.scale_pre, base.scale_mid, base.scale_post)
    x = syn.synthetic_activations(3, 4096, seed=1).to(dev)
    for compact in (mixed, _product_fixture(True)):
        xs = x if compact is mixed else syn.synthetic_activations(2, 35, seed=2, dtype=torch.float32).to(dev)
        y_compact = backend.linear(xs, backend.prepare(compact, dev))
        y_packed = backend.linear(xs, backend.prepare(compact.to_packed(), dev))
        assert torch.equal(y_compact, y_packed)
