"""The C-ABI library loads and exports every entry point include/*.h declares.
No compute call is made here (no GPU needed)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

from nanoquant_amd.runtime import _native

HEADERS = sorted((Path(__file__).resolve().parent.parent / "include").glob("*.h"))


def _declared_functions() -> set[str]:
    names: set[str] = set()
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(nq_[a-z0-9_]+)\s*\(", text))
    return names


def test_header_and_binding_agree():
    assert _declared_functions() == set(_native.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = _native.load()
    for name in _declared_functions():
        assert hasattr(lib, name), name


def test_host_only_entry_points():
    lib = _native.load()
    assert lib.nq_abi_version() == 3
    assert _native.status_text(-5).startswith("workspace smaller")
    # Argument validation happens before any device work.
    desc = _native.LinearDesc()
    assert lib.nq_linear_workspace_bytes(ctypes.byref(desc), 1) == -1
    assert lib.nq_linear(ctypes.byref(desc), None, 0, 1, None, 0, None, 0, None) == _native.NQ_ERR_SHAPE
    assert lib.nq_unpack_signs(None, 1, 1, 1, 0, None, None) == _native.NQ_ERR_ARGUMENT


def test_tile_layout_restatement_is_a_bit_permutation():
    """The numpy tile layout (checked word for word against the GPU builder in
    the GPU tests) moves every sign bit to exactly one place: decoding it with
    the inverse map recovers the matrix, including word and row tails."""

    import numpy as np

    from tile_layout import build_tiles, geometry, sign_bits

    rng = np.random.default_rng(5)
    for rows, cols in [(16, 128), (33, 819), (5, 7), (40, 1536)]:
        words = rng.integers(-(2**31), 2**31, size=(rows, -(-cols // 32)), dtype=np.int64).astype(np.int32)
        if cols % 32:
            words[:, -1] &= (1 << (cols % 32)) - 1
        tiles = build_tiles(words, rows, cols)
        nt, nb, _ = geometry(rows, cols)
        got = np.zeros((nt * 16, nb * 128), dtype=np.uint32)
        for k in range(nb * 128):
            c, d, m, g, b = k // 512, (k // 128) % 4, (k // 16) % 8, (k // 4) % 4, k % 4
            dw = min(4, nb - 4 * c)
            for r in range(nt * 16):
                t, n = divmod(r, 16)
                w = tiles[t * nb * 64 + c * 256 + (16 * g + n) * dw + d]
                got[r, k] = (int(w) >> (8 * b + m)) & 1
        expected = np.zeros_like(got)
        expected[:rows, :cols] = sign_bits(words, rows, cols)
        np.testing.assert_array_equal(got, expected)
        assert int(np.unpackbits(tiles.view(np.uint8)).sum()) == int(expected.sum())
