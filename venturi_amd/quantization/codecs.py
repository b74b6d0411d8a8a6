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
    """CPU reference decode of stored planes to fp16 (codecs.py:144-177).

    Rejects non-finite or negative scales and, for Q8, the forbidden code -128.
    """
    codec = codec_for(fmt)
    n, k = shape
    if not codec.quantized:
        raise ValueError("Expected a quantized codec")
    groups = (-(-k // 128) * 128) // codec.group
    plane = codes.numpy().reshape(n, groups, 32)
    scale = scales.numpy().reshape(n, groups).astype(np.float32)
    if not np.isfinite(scale).all() or (scale < 0).any():
        raise ValueError("Invalid stored scale")
    if codec.bits == 8:
        if (plane == -128).any():
            raise ValueError("Forbidden Q8 code")
        signed = plane.astype(np.float32)
    else:
        lanes = np.empty((n, groups, 64), dtype=np.int32)
        lanes[:, :, 0::2] = plane & 15
        lanes[:, :, 1::2] = plane >> 4
        if codec.high_plane:
            extra = codec.bits - 4
            if high is None:
                raise ValueError("Missing high-bit plane")
            hi = high.numpy().reshape(n, groups, 8 * extra)
            for lane in range(64):
                bits = (hi[:, :, lane * extra // 8] >> (lane * extra % 8)) & ((1 << extra) - 1)
                lanes[:, :, lane] |= bits.astype(np.int32) << 4
        half_range = 1 << (codec.bits - 1)
        signed = np.where(lanes >= half_range, lanes - (1 << codec.bits), lanes).astype(np.float32)
    values = (signed * scale[:, :, None]).reshape(n, -1)[:, :k]
    return torch.from_numpy(np.ascontiguousarray(values)).to(torch.float16)
