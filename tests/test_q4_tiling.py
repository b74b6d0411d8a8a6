"""The tiled decode copy of Q4 planes (q4.tile_q4), checked byte by byte on the CPU.

Lane (r, q) of row block b, chunk c must hold the 16 code bytes of row
16b + r at bytes 64c + 16q of the row-major plane, and the scale slot (b, c, r)
the two group scales 2c, 2c + 1 of that row; rows past n are zero.
"""

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
                    want = codes[row, 64 * c + 16 * q: 64 * c + 16 * q + 16] if row < n else np.zeros(16, np.uint8)
                    assert np.array_equal(tc[b, c, q, r], want)
            for r in range(16):
                row = 16 * b + r
                want = scales[row, 2 * c: 2 * c + 2] if row < n else np.zeros(2, np.float16)
                assert np.array_equal(ts[b, c, r], want)
    # The flat order is the kernel's: [block][chunk][lane 16q + r][16 bytes].
    flat = tc.reshape(-1)
    b, c, q, r = blocks - 1, chunks - 1, 3, min(15, n - 1 - 16 * (blocks - 1))
    off = ((b * chunks + c) * 64 + 16 * q + r) * 16
    assert np.array_equal(flat[off:off + 16], codes[16 * b + r, 64 * c + 48: 64 * c + 64])
