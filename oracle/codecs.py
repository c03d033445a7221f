"""CPU oracle for the prepare-time right-factor codecs — TEST INFRASTRUCTURE ONLY
(imported by tests/ only; the product decodes on the device).

Restates, in numpy integer arithmetic:

* mixed-V ``mixed-v-free-k10-pair9-v1`` (src/nanoquant/runtime/mixed_v.py:18-146):
  the right factor's first ``free_rows`` rows are canonical sign words; every
  remaining word is one 19-bit record (10-bit codebook index in the low bits,
  9-bit pair id above), records packed LSB-first into int32 words with zero
  padding; the word is ``codebook[index] ^ (1 << a | 1 << b)`` where pair id
  enumerates ``(a, b), a < b < 32`` lexicographically (496 valid ids);
* product codebook ``product-codebook-free-k16-v1``
  (src/nanoquant/runtime/product_codebook.py:27-128): coded words are 16-bit
  indices packed two per int32 (low half first, a zero padding record when
  odd); the word is ``first[i & 0xFF] | second[i >> 8] << 16`` with two
  256-entry 16-bit half-word tables;
* the packed sign-matrix transpose used for transposed factorizations
  (src/nanoquant/runtime/product_codebook.py:232-250).

Pinned by the reference tests' known answers (tests/unit/test_runtime_mixed_v.py:32-46,
tests/unit/test_runtime_product_codebook.py:62-73: payload sizes, round trips,
the padding and pair-id rejections, the decoded fixture words) and by
brute-force bit-by-bit evaluation in tests/test_codecs.py.
"""

from __future__ import annotations

import numpy as np

MIXED_V_INDEX_BITS = 10
MIXED_V_PAIR_BITS = 9
MIXED_V_RECORD_BITS = 19
MIXED_V_PAIRS = 496
PRODUCT_INDEX_BITS = 16


def pair_bits(pair_id: int) -> tuple[int, int]:
    """The (a, b), a < b, of a lexicographic pair id over 32 bit positions."""

    for a in range(32):
        run = 31 - a
        if pair_id < run:
            return a, a + 1 + pair_id
        pair_id -= run
    raise ValueError("pair id outside the 496 pairs")


def payload_words(records: int, bits: int) -> int:
    return (records * bits + 31) // 32


def pack_records(values: np.ndarray, bits: int) -> np.ndarray:
    """Row-major records of `bits` bits, LSB-first, into uint32 words."""

    flat = np.asarray(values, dtype=np.uint64).reshape(-1)
    out = np.zeros(payload_words(flat.size, bits), dtype=np.uint64)
    for i, v in enumerate(flat.tolist()):
        pos = i * bits
        out[pos // 32] |= (v << (pos % 32)) & 0xFFFFFFFF
        if pos % 32 + bits > 32:
            out[pos // 32 + 1] |= v >> (32 - pos % 32)
    return out.astype(np.uint32).view(np.int32)


def unpack_records(payload: np.ndarray, count: int, bits: int) -> np.ndarray:
    words = np.asarray(payload).view(np.uint32).astype(np.uint64)
    out = np.zeros(count, dtype=np.uint64)
    for i in range(count):
        pos = i * bits
        v = words[pos // 32] >> np.uint64(pos % 32)
        if pos % 32 + bits > 32:
            v |= words[pos // 32 + 1] << np.uint64(32 - pos % 32)
        out[i] = v & np.uint64((1 << bits) - 1)
    return out


def decode_mixed_v(free_words: np.ndarray, payload: np.ndarray, codebook: np.ndarray, rank: int,
                   words_per_row: int) -> tuple[np.ndarray, int]:
    """Canonical right words [rank, words_per_row] and the count of invalid pair ids
    (those words decode as codebook[index] unchanged)."""

    free = np.asarray(free_words).view(np.uint32)
    coded_rows = rank - free.shape[0]
    records = unpack_records(payload, coded_rows * words_per_row, MIXED_V_RECORD_BITS)
    book = np.asarray(codebook).view(np.uint32)
    out = np.zeros((rank, words_per_row), dtype=np.uint32)
    out[: free.shape[0]] = free
    bad = 0
    for i, rec in enumerate(records.tolist()):
        index, pair = rec & 1023, rec >> 10
        word = int(book[index])
        if pair < MIXED_V_PAIRS:
            a, b = pair_bits(pair)
            word ^= (1 << a) | (1 << b)
        else:
            bad += 1
        out[free.shape[0] + i // words_per_row, i % words_per_row] = word
    return out.view(np.int32), bad


def decode_product_codebook(free_words: np.ndarray, payload: np.ndarray, first: np.ndarray, second: np.ndarray,
                            rank: int, words_per_row: int) -> np.ndarray:
    free = np.asarray(free_words).view(np.uint32)
    coded_rows = rank - free.shape[0]
    indices = unpack_records(payload, coded_rows * words_per_row, PRODUCT_INDEX_BITS).astype(np.int64)
    lo = np.asarray(first).view(np.uint16).astype(np.uint32)
    hi = np.asarray(second).view(np.uint16).astype(np.uint32)
    coded = lo[indices & 0xFF] | (hi[indices >> 8] << np.uint32(16))
    return np.concatenate([free, coded.reshape(coded_rows, words_per_row)]).view(np.int32)


def transpose_signs(words: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Packed words of the transposed sign matrix, bit by bit."""

    src = np.asarray(words).view(np.uint32)
    out = np.zeros((cols, (rows + 31) // 32), dtype=np.uint32)
    for r in range(rows):
        for c in range(cols):
            if (int(src[r, c // 32]) >> (c % 32)) & 1:
                out[c, r // 32] |= np.uint32(1 << (r % 32))
    return out.view(np.int32)
