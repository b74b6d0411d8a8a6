"""Q4 (q4_g64_fp16) codec helpers and the W4A16 linear plan.

``quantize_q4_rtn`` and ``decode_q4_fp16`` mirror the reference's expert codec
(models/flash_next/flash_next_q4.py:26-62): fp16 scale = fp16(max|w|/7)
floored at 2^-24, codes = clamp(round_half_even(w / scale), -7, 7), and the
W4A16 weight value fp16(q * scale).
"""

import torch
from torch.nn import functional as F

from .weights import Q4RowSplitWeight


def quantize_q4_rtn(weight, *, max_elements=16 * 2**20):
    """CPU round-to-nearest-even Q4 with the fp16 scale rounded before the codes."""
    if (
        not isinstance(weight, torch.Tensor)
        or weight.device.type != "cpu"
        or weight.ndim != 2
        or weight.dtype not in (torch.float16, torch.bfloat16, torch.float32)
        or min(weight.shape) < 1
    ):
        raise ValueError("Explicit nonempty CPU floating weight required")
    if type(max_elements) is not int or max_elements <= 0 or weight.numel() > max_elements:
        raise ValueError("Q4 quantization exceeds explicit element budget")
    value = weight.float()
    if not torch.isfinite(value).all():
        raise ValueError("Finite source weights required")
    rows, cols = weight.shape
    padded = (cols + 127) // 128 * 128
    blocks = F.pad(value, (0, padded - cols)).reshape(rows, padded // 64, 64)
    scales = (blocks.abs().amax(-1) / 7).clamp_min(2**-24).half()
    if not torch.isfinite(scales).all():
        raise ValueError("Source scale overflows FP16")
    codes = (blocks / scales.float().unsqueeze(-1)).round().clamp(-7, 7).to(torch.int8)
    if not torch.isfinite((codes.float() * scales.float().unsqueeze(-1)).half()).all():
        raise ValueError("Quantized weight overflows FP16 execution")
    return Q4RowSplitWeight.from_codes(codes.reshape(rows, padded)[:, :cols], scales[:, : (cols + 63) // 64])


def decode_q4_fp16(weight):
    """fp16 matrix of fp16(q * scale) values (diagnostic; no retained cache)."""
    weight.validate()
    nibbles = torch.stack((weight.codes & 15, weight.codes >> 4), -1).reshape(weight.out_features, weight.padded_k)
    nibbles = nibbles.to(torch.int16)
    signed = torch.where(nibbles < 8, nibbles, nibbles - 16)
    values = signed.float().reshape(weight.out_features, -1, 64) * weight.scales.float().unsqueeze(-1)
    return values.reshape(weight.out_features, -1)[:, : weight.in_features].half()


def upload_q4(backend, weight, *, device, dtype):
    raise NotImplementedError("Q4 linear kernels are not in this build yet")
