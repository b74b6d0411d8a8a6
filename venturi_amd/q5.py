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


# Bit offsets of the four column pairs of an 8-column word inside its 16-bit
# half of a high-plane register: pairs (c, c+1), (c+2, c+3), (c+4, c+5),
# (c+6, c+7) of word jj of the register sit at hb * jj plus these.
_PAIR_OFFSETS = (0, 8, 4, 12)


def tile_row_codec(codes, high, scales, bits):
    """Tiled decode copy of q5_g64 / q6_g64 planes (read by ``venturi_row_tiled_run``).

    Codes [row block][chunk][lane l = 16q + r][16 bytes] as for Q4 (row r of the
    16-row block, columns 128c + 32q .. +32 of the chunk, four 4-byte words of
    8 columns) with the low nibbles as stored (no bias) in Q4's tiled order:
    nibble j of a word holds column c + 2j, nibble 4 + j column c + 2j + 1.
    High plane [row block][chunk][lane][hb 4-byte registers] (hb = bits - 4):
    each column's upper hb bits biased (the sign bit flipped, so nibble and
    upper bits form the code plus 2^(bits - 1)); register i holds words
    jj = 0 .. 4/hb - 1 of the lane (word 4i/hb + jj), the pair (c + 2m,
    c + 2m + 1) of word jj at bits hb * jj + (0, 8, 4, 12)[m] and 16 above.
    Scales [row block][chunk][r][2]. Rows past n are zero.
    """
    if bits not in (5, 6):
        raise ValueError("tile_row_codec takes 5- or 6-bit planes")
    hb = bits - 4
    n, row_bytes = codes.shape
    padded = 2 * row_bytes
    chunks = row_bytes // 64
    blocks = (n + 15) // 16
    device = codes.device
    nib = torch.stack((codes & 15, codes >> 4), -1).reshape(n, padded // 8, 8)
    nib = nib[:, :, [0, 2, 4, 6, 1, 3, 5, 7]].reshape(n, row_bytes, 2)
    packed = nib[..., 0] | (nib[..., 1] << 4)
    # Upper bits per column from the LSB-first stream, then biased.
    stream = (high.unsqueeze(-1) >> torch.arange(8, dtype=torch.uint8, device=device)) & 1
    stream = stream.reshape(n, padded, hb).to(torch.int64)
    upper = sum(stream[..., b] << b for b in range(hb)) ^ (1 << (hb - 1))
    upper = upper.view(n, chunks, 4, 4, 8)  # [row][chunk][q][word][column]
    per = 4 // hb  # words per register
    words = torch.arange(4, device=device)
    offset = (hb * (words % per))[:, None] + torch.tensor(_PAIR_OFFSETS, device=device)[None, :]  # [word][pair]
    fields = (upper[..., 0::2] << offset) | (upper[..., 1::2] << (offset + 16))
    regs = fields.sum(-1).view(n, chunks, 4, hb, per).sum(-1)  # disjoint bits: sums are ors
    regs = (regs - ((regs >> 31) << 32)).to(torch.int32)  # the same 32 bits as int32
    c = torch.zeros((blocks * 16, row_bytes), dtype=torch.uint8, device=device)
    h = torch.zeros((blocks * 16, chunks * 16 * hb), dtype=torch.uint8, device=device)
    s = torch.zeros((blocks * 16, chunks * 2), dtype=torch.float16, device=device)
    c[:n] = packed
    h[:n] = regs.reshape(n, chunks * 4 * hb).view(torch.uint8)
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
