"""Row-codec geometry shared by every format in the registry.

Mirrors venturi.quantization.layout (reference layout.py:3-39): each row of an
[N, K] matrix is padded to a multiple of 128 columns, split into groups of
``group`` columns, and stored as a 32-byte base plane per group (plus a high
plane for 5/6-bit codes) and one fp16 scale per group.
"""

ROW_FORMATS = {
    "q4_g64_fp16": (4, 64),
    "q5_g64_fp16": (5, 64),
    "q6_g64_fp16": (6, 64),
    "q8_g32_fp16": (8, 32),
}


def _round_up(value, multiple=256):
    return -(-value // multiple) * multiple


def row_geometry(shape, format):
    """Device-local plane offsets: (bits, group, groups, high_offset, scales_offset, total).

    Planes start on 256-byte boundaries; this is scratch geometry, not a file
    layout (layout.py:15-31).
    """
    n, k = shape
    bits, group = ROW_FORMATS[format]
    groups = _round_up(k, 128) // group
    base = n * groups * 32
    high = n * groups * 8 * (bits - 4) if bits in (5, 6) else 0
    high_offset = _round_up(base)
    scales_offset = high_offset + _round_up(high)
    return bits, group, groups, high_offset, scales_offset, scales_offset + n * groups * 2


def row_payload_bytes(shape, format):
    """Bytes of codes, high bits and scales with no alignment padding (layout.py:34-39)."""
    n, k = shape
    bits, group = ROW_FORMATS[format]
    padded = _round_up(k, 128)
    return n * (padded * bits // 8 + padded // group * 2)
