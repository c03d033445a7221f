"""numpy restatement of the GPU tile layout written by ``nq_prepare_tiles``.

The layout is this package's own (not the reference's); the GPU tests compare
the device builder against this function word for word. A sign matrix
[rows, cols] is cut into 16-row tiles and 512-column chunks (the last chunk
128, 256, 384 or 512 columns wide). Lane ``l = 16*g + n`` of tile ``t`` owns row
``16*t + n``; in chunk ``c`` it has ``dw = min(4, nb - 4*c)`` words stored
contiguously, and bit ``8*b + m`` of its word ``d`` is the sign bit (1 = -1) of
column ``512*c + 128*d + 16*m + 4*g + b``. Bits past ``rows`` or ``cols`` are 0.
"""

from __future__ import annotations

import numpy as np


def geometry(rows: int, cols: int) -> tuple[int, int, int]:
    nt = -(-rows // 16)
    nb = -(-cols // 128)
    nc = -(-nb // 4)
    return nt, nb, nc


def sign_bits(words: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Canonical llama.cpp-i32-lsb-v1 words [rows, ceil(cols/32)] -> bits [rows, cols]."""

    w = np.ascontiguousarray(words, dtype=np.int32).view(np.uint32).reshape(rows, -1)
    bits = (w[:, :, None] >> np.arange(32, dtype=np.uint32)) & 1
    return bits.reshape(rows, -1)[:, :cols].astype(np.uint32)


def build_tiles(words: np.ndarray, rows: int, cols: int) -> np.ndarray:
    nt, nb, nc = geometry(rows, cols)
    bits = np.zeros((nt * 16, nb * 128), dtype=np.uint32)
    bits[:rows, :cols] = sign_bits(words, rows, cols)
    out = np.zeros(nt * nb * 64, dtype=np.uint32)
    lanes = np.arange(64)
    n, g = lanes % 16, lanes // 16
    for t in range(nt):
        row = 16 * t + n
        for c in range(nc):
            dw = min(4, nb - 4 * c)
            for d in range(dw):
                word = np.zeros(64, dtype=np.uint32)
                for m in range(8):
                    for b in range(4):
                        col = 512 * c + 128 * d + 16 * m + 4 * g + b
                        word |= bits[row, col] << np.uint32(8 * b + m)
                out[t * nb * 64 + c * 256 + lanes * dw + d] = word
    return out
