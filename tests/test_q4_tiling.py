"""The tiled decode copy of Q4 planes (q4.tile_q4), checked byte by byte on the CPU.

Lane (r, q) of row block b, chunk c must hold the codes of row 16b + r at
bytes 64c + 16q of the row-major plane, each 4-byte word re-packed as biased
nibbles (q + 8) with nibble j = column 2j and nibble 4 + j = column 2j + 1 of
its eight columns; the scale slot (b, c, r) holds the two group scales 2c,
2c + 1 of that row; rows past n are zero.
"""


def expected_word_bytes(raw):
    """Scalar restatement of the word re-packing for 16 row-major code bytes."""
    out = np.zeros(16, np.uint8)
    for w in range(4):
        cols = []
        for b in range(4):
            byte = int(raw[4 * w + b])
            cols += [byte & 15, byte >> 4]  # columns 2b, 2b + 1
        nibbles = [cols[0], cols[2], cols[4], cols[6], cols[1], cols[3], cols[5], cols[7]]
        nibbles = [v ^ 8 for v in nibbles]  # q + 8 for the two's complement nibble q
        for b in range(4):
            out[4 * w + b] = nibbles[2 * b] | (nibbles[2 * b + 1] << 4)
    return out

import numpy as np
import pytest
import torch

from venturi_amd.q4 import tile_q4


@pytest.mark.parametrize("n,row_bytes", [(1, 64), (16, 128), (37, 192), (130, 1024)])
def test_tile_q4_layout(n, row_bytes):
    rng = np.random.default_rng(n + row_bytes)
    codes = rng.integers(0, 256, size=(n, row_bytes), dtype=np.uint8)
    scales = rng.random((n, row_bytes // 32)).astype(np.float16)
    tc, ts = tile_q4(torch.from_numpy(codes), torch.from_numpy(scales))
    blocks, chunks = (n + 15) // 16, row_bytes // 64
    assert tc.shape == (blocks, chunks, 4, 16, 16) and ts.shape == (blocks, chunks, 16, 2)
    tc, ts = tc.numpy(), ts.numpy()
    for b in range(blocks):
        for c in range(chunks):
            for q in range(4):
                for r in range(16):
                    row = 16 * b + r
                    want = (expected_word_bytes(codes[row, 64 * c + 16 * q: 64 * c + 16 * q + 16]) if row < n
                            else np.zeros(16, np.uint8))
                    assert np.array_equal(tc[b, c, q, r], want)
            for r in range(16):
                row = 16 * b + r
                want = scales[row, 2 * c: 2 * c + 2] if row < n else np.zeros(2, np.float16)
                assert np.array_equal(ts[b, c, r], want)
    # The flat order is the kernel's: [block][chunk][lane 16q + r][16 bytes].
    flat = tc.reshape(-1)
    b, c, q, r = blocks - 1, chunks - 1, 3, min(15, n - 1 - 16 * (blocks - 1))
    off = ((b * chunks + c) * 64 + 16 * q + r) * 16
    assert np.array_equal(flat[off:off + 16], expected_word_bytes(codes[16 * b + r, 64 * c + 48: 64 * c + 64]))


def test_biased_nibble_values():
    # Biased nibble u = q + 8 for the two's complement nibble q: 0 -> 8, 7 -> 15, -8 (0x8) -> 0, -1 (0xF) -> 7.
    codes = torch.tensor([[0x70, 0xF8] + [0] * 62], dtype=torch.uint8)
    tc, _ = tile_q4(codes, torch.zeros(1, 2, dtype=torch.float16))
    word = tc.reshape(-1)[:4].numpy()
    # columns: c0 = 0, c1 = 7, c2 = -8, c3 = -1, c4..c7 = 0 -> nibbles [c0, c2, c4, c6, c1, c3, c5, c7] + 8
    # = [8, 0, 8, 8, 15, 7, 8, 8], two per byte, low nibble first
    assert list(word) == [0x08, 0x88, 0x7F, 0x88]
