"""Weight codec registry and per-architecture qualification tables.

Mirrors venturi.quantization.codecs (reference codecs.py:24-194): the same
``Codec`` record, ``CODECS`` table, ``codec_for`` lookup and CPU reference
``dequantize_planes``. The qualification tables keep the reference's keys and
add this build's gfx950 entry (torch on ROCm reports MI355X as capability
(9, 5)); Q8 and Q4 are the formats executed by this library.
"""

from dataclasses import dataclass

import numpy as np
import torch

from .layout import ROW_FORMATS, row_payload_bytes

DENSE_ITEMSIZE = {"fp16": 2, "bf16": 2, "fp32": 4}

GFX950 = (9, 5)


@dataclass(frozen=True)
class Codec:
    fmt: str
    layout: str
    bits: int = 0
    group: int = 0
    scale_dtype: str = ""
    high_plane: bool = False
    dense: bool = False
    forbidden_codes: tuple = ()

    @property
    def quantized(self) -> bool:
        return self.layout == "row_split_k128_v1"

    def encoded_bytes(self, n: int, k: int) -> int:
        if self.dense:
            return n * k * DENSE_ITEMSIZE[self.fmt]
        return row_payload_bytes((n, k), self.fmt)

    def upload_bytes(self, n: int, k: int) -> int:
        """Resident bytes: code and scale planes without inter-plane padding."""
        if self.dense:
            return n * k * DENSE_ITEMSIZE[self.fmt]
        padded = -(-k // 128) * 128
        return n * (padded * self.bits // 8 + padded // self.group * 2)


def _row_codec(fmt):
    bits, group = ROW_FORMATS[fmt]
    return Codec(
        fmt=fmt,
        layout="row_split_k128_v1",
        bits=bits,
        group=group,
        scale_dtype="fp16",
        high_plane=bits in (5, 6),
        forbidden_codes=(-128,) if bits == 8 else (),
    )


CODECS = {fmt: _row_codec(fmt) for fmt in ROW_FORMATS}
CODECS.update(
    {fmt: Codec(fmt=fmt, layout="contiguous_le_v1", dense=True) for fmt in ("fp16", "bf16", "fp32")}
)

# Execution qualification per architecture. The NVIDIA keys are the
# reference's; GFX950 lists the codecs this library executes and tests.
EXECUTION_QUALIFIED = {
    (7, 0): {"q8_g32_fp16", "q5_g64_fp16"},
    (8, 9): {"q8_g32_fp16", "q4_g64_fp16", "q5_g64_fp16", "q6_g64_fp16"},
    (8, 6): {"q8_g32_fp16"},
    GFX950: {"q8_g32_fp16", "q4_g64_fp16"},
}

# One-pass int8 activations are a separate model-quality gate (codecs.py:180-183);
# the kernels exist here, the model qualification does not.
ACTIVATION_INT8_QUALIFIED = {(7, 0): set(), (8, 9): set(), GFX950: set()}

FUSED_LINEAR_QUALIFIED = {
    (7, 0): {"q8_g32_fp16"},
    (8, 9): {"q8_g32_fp16"},
    GFX950: {"q8_g32_fp16"},
}


def codec_for(fmt: str) -> Codec:
    try:
        return CODECS[fmt]
    except KeyError:
        raise ValueError(f"Unknown weight format {fmt!r}; registered: {sorted(CODECS)}") from None


def dequantize_planes(codes, scales, high, shape, fmt):
    """CPU decode of stored planes to fp16 (the reference's is codecs.py:105-139).

    Written from the plane layout: a row's padded columns (k rounded up to 128)
    carry one code each; Q8 stores them as int8 (-128 is forbidden), the 4-bit
    body of Q4/Q5/Q6 packs column 2j in the low nibble of byte j and 2j + 1 in
    the high nibble, and Q5/Q6 keep the upper bits of column c at bit offset
    c * (bits - 4) of the row's high plane (least significant bit first). The
    code is the two's complement of its bits; the weight is code * scale of
    the column's group. Rejects non-finite or negative scales.
    """
    codec = codec_for(fmt)
    if not codec.quantized:
        raise ValueError("Expected a quantized codec")
    rows, cols = shape
    padded = -(-cols // 128) * 128
    scale = scales.numpy().astype(np.float32).reshape(rows, padded // codec.group)
    if not np.isfinite(scale).all() or (scale < 0).any():
        raise ValueError("Invalid stored scale")
    code = _column_codes(codec, codes.numpy().reshape(rows, -1), high, rows, padded)
    weight = code.astype(np.float32) * np.repeat(scale, codec.group, axis=1)
    return torch.from_numpy(np.ascontiguousarray(weight[:, :cols])).to(torch.float16)


def _column_codes(codec, plane, high, rows, padded):
    """Signed integer code of every padded column, [rows, padded] int32."""
    if codec.bits == 8:
        if (plane == -128).any():
            raise ValueError("Forbidden Q8 code")
        return plane.astype(np.int32)
    body = plane.view(np.uint8)
    code = np.empty((rows, padded), dtype=np.int32)
    code[:, 0::2] = body & 0x0F
    code[:, 1::2] = body >> 4
    if codec.high_plane:
        if high is None:
            raise ValueError("Missing high-bit plane")
        extra = codec.bits - 4
        bits = np.unpackbits(high.numpy().view(np.uint8).reshape(rows, -1), axis=1, bitorder="little")
        upper = bits[:, : padded * extra].reshape(rows, padded, extra).astype(np.int32) @ (1 << np.arange(extra))
        code |= upper << 4
    return code - ((code >> (codec.bits - 1)) << codec.bits)
