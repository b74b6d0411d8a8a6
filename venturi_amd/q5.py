"""Q5 (q5_g64_fp16) codec helpers and the W5A16 operator object.

``quantize_q5_rtn`` and ``decode_q5_fp16`` mirror the reference's experimental
W5A16 codec (models/flash_next/flash_next_q5.py:19-70): fp16 scale =
fp16(max|w|/15) floored at 2^-24 and rounded before the codes, codes =
round_half_even(w / scale) in [-16, 15] (a +16 produced by the scale rounding
saturates to +15), and the W5A16 weight value fp16(q * scale). ``NativeQ5``
mirrors ops/flash_next_q5.py over this library's Q5 ABI 1 with gfx950
qualification instead of SM70.
"""

from dataclasses import dataclass

import torch

from .plugin import CodecEntry, RowCodecOperator
from .weights import Q5RowSplitWeight, decode_k64_fp16, rtn_k64

CODEC = "rtn_symmetric15_g64_fp16_row_split_k128_v1"


def quantize_q5_rtn(weight, *, max_elements=16 * 2**20):
    """CPU RTN for the experimental W5A16 codec (flash_next_q5.py:18-50): per K64 group the
    fp16 scale fp16(max(max|w| / 15, 2^-24)) is rounded first, then q = RNE(w / scale) in
    [-16, 15] (a +16 from the scale's rounding saturates to 15); returns a ``Q5RowSplitWeight``."""
    codes, scales = rtn_k64(weight, levels=15, lowest=-16, tag="Q5", max_elements=max_elements)
    return Q5RowSplitWeight.from_codes(codes, scales)


def tile_row_codec(codes, high, scales, bits):
    """Tiled decode copy of q5_g64 / q6_g64 planes (read by ``venturi_row_tiled_run``).

    Codes [row block][chunk][lane l = 16q + r][16 bytes] as for Q4 (row r of the
    16-row block, code bytes 16q .. 16q+15 of the 128-column chunk) but with the
    row-major nibbles; high plane [row block][chunk][lane][4 * hb bytes] (the
    lane's 32 columns' upper hb = bits - 4 bits, LSB-first as in the row-major
    stream); scales [row block][chunk][r][2]. Rows past n are zero.
    """
    if bits not in (5, 6):
        raise ValueError("tile_row_codec takes 5- or 6-bit planes")
    hb = bits - 4
    n, row_bytes = codes.shape
    chunks = row_bytes // 64
    blocks = (n + 15) // 16
    c = torch.zeros((blocks * 16, row_bytes), dtype=torch.uint8, device=codes.device)
    h = torch.zeros((blocks * 16, chunks * 16 * hb), dtype=torch.uint8, device=codes.device)
    s = torch.zeros((blocks * 16, chunks * 2), dtype=torch.float16, device=codes.device)
    c[:n] = codes
    h[:n] = high
    s[:n] = scales
    tc = c.view(blocks, 16, chunks, 4, 16).permute(0, 2, 3, 1, 4).contiguous()
    th = h.view(blocks, 16, chunks, 4, 4 * hb).permute(0, 2, 3, 1, 4).contiguous()
    ts = s.view(blocks, 16, chunks, 2).permute(0, 2, 1, 3).contiguous()
    return tc, th, ts


def decode_q5_fp16(weight):
    """fp16 matrix of fp16(q * scale) values, the W5A16 weights (diagnostic; no retained cache)."""
    return decode_k64_fp16(weight, 5)


@dataclass(frozen=True)
class PreparedQ5:
    weight: Q5RowSplitWeight
    ready: object


class NativeQ5(RowCodecOperator):
    """W5A16 operators of Q5 ABI 1 (reference ops/flash_next_q5.py:17-89).

    ``linear`` is the reference GEMV order (fp16(q*scale) weights,
    lane-strided fmaf, 32-lane tree) for 1..64 fp16 tokens; ``decode`` writes
    the fp16 matrix.
    """

    entry = CodecEntry("Q5", Q5RowSplitWeight, ("codes", "high", "scales"), "venturi_q5_abi", "venturi_q5_decode",
                       "venturi_q5_linear")
    prepared = PreparedQ5
