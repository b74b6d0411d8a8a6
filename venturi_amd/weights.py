"""Weight descriptors: dense, and the Q4 / Q5 / Q8 row-split codecs.

The public surface is the reference's (src/venturi/ops/weights.py:8-454): the
classes, field names, ``format`` / ``layout`` / ``group_size`` tags, the
``validate``, ``from_codes``, ``from_payload``, ``from_dense`` and
``dequantize_reference`` methods and their error texts, so a descriptor built
by either library describes the same bytes:

* Q8 (``q8_g32_fp16``): codes int8 [N, Kp] in [-127, 127], scales fp16
  [N, Kp/32]; value = code * scale.
* Q4 (``q4_g64_fp16``): codes uint8 [N, Kp/2] holding two's-complement
  nibbles (column 2j in the low nibble of byte j), scales fp16 [N, Kp/64].
* Q5 (``q5_g64_fp16``): Q4's nibble plane for the low four bits, plus a high
  plane uint8 [N, Kp/8] with the fifth bit of column c at bit c % 8 of byte
  c // 8; codes in [-16, 15].

Kp = ceil(K/128)*128; padding columns hold code 0 and padding groups scale 0.

Here the nibble codecs state their extra planes as data (``_extra_planes``)
and each validator is an ordered rule table (``_raise_first``); the float encoders share one group round-to-nearest-even
routine (``_rtn_codes``) and the bit packers operate on whole planes.
"""

from dataclasses import dataclass

import torch

_INT32 = 2**31
_SIGNED = (torch.int8, torch.int16, torch.int32, torch.int64)
_FLOATS = (torch.float16, torch.bfloat16, torch.float32, torch.float64)


def _padded(k):
    return (k + 127) // 128 * 128


def _int32_extent(value):
    return type(value) is int and 0 < value < _INT32


def _raise_first(rules):
    """Raises the error of the first failed rule; rules are (failed, type, message), `failed` a callable."""
    for failed, error, message in rules:
        if failed():
            raise error(message)


# ---------------------------------------------------------------- bit planes


def _nibbles(values):
    """uint8 [N, C/2]: the low four bits of column 2j in the low nibble of byte j."""
    low = (values & 15).to(torch.uint8)
    pairs = low.view(values.shape[0], -1, 2)
    return (pairs[..., 0] | (pairs[..., 1] << 4)).contiguous()


def _unnibble(codes):
    """int16 [N, 2 * bytes]: the nibbles of a plane in column order (unsigned)."""
    return torch.stack((codes & 15, codes >> 4), dim=-1).reshape(codes.shape[0], -1).to(torch.int16)


def _bitplane(bit):
    """uint8 [N, C/8] from a 0/1 plane [N, C]: column c at bit c % 8 of byte c // 8."""
    weights = torch.tensor([1 << i for i in range(8)], dtype=torch.int16)
    return (bit.to(torch.int16).view(bit.shape[0], -1, 8) * weights).sum(-1).to(torch.uint8).contiguous()


def _unbitplane(plane):
    shifts = torch.arange(8, dtype=torch.int16)
    return ((plane.to(torch.int16).unsqueeze(-1) >> shifts) & 1).reshape(plane.shape[0], -1)


def _signed(unsigned, bits):
    half = 1 << (bits - 1)
    return torch.where(unsigned < half, unsigned, unsigned - 2 * half)


def _group_values(signed, scales, group, in_features):
    """FP64 q * scale over columns [0, in_features)."""
    return (signed.to(torch.float64) * scales.to(torch.float64).repeat_interleave(group, 1))[:, :in_features]


# ---------------------------------------------------------------- float encoders


def _rtn_codes(source, *, group, levels, lowest, name, rows_per_chunk, code_dtype):
    """Per-group nearest-even quantization with the stored fp16 scale.

    scale = fp16(max|group| / levels) in the working precision (f32, or f64
    for f64 sources); code = clamp(round_half_even(x / scale), lowest,
    levels), or 0 where the stored scale is 0 (true division, as the reference
    divides). Returns codes [N, Kp] and scales [N, Kp / group] over the
    zero-padded K; rejects non-finite sources and scales that overflow fp16.
    """
    dense = DenseWeight(source)
    if source.device.type != "cpu":
        raise ValueError(f"{name} quantization requires an explicit CPU source")
    if not _int32_extent(rows_per_chunk):
        raise ValueError("rows_per_chunk must be a positive int32")
    n, k = dense.out_features, dense.in_features
    padded = _padded(k)
    if padded >= _INT32:
        raise ValueError(f"Padded {name} K must fit int32")
    work = torch.float64 if source.dtype == torch.float64 else torch.float32
    codes = torch.zeros(n, padded, dtype=code_dtype)
    scales = torch.zeros(n, padded // group, dtype=torch.float16)
    with torch.no_grad():
        for first in range(0, n, rows_per_chunk):
            rows = slice(first, min(n, first + rows_per_chunk))
            block = torch.nn.functional.pad(source[rows].detach().to(work), (0, padded - k))
            if not bool(torch.isfinite(block).all()):
                raise ValueError(f"{name} source must be finite")
            grouped = block.view(block.shape[0], -1, group)
            stored = (grouped.abs().amax(-1) / levels).to(torch.float16)
            if not bool(torch.isfinite(stored).all()):
                raise ValueError(f"{name} group scale overflows FP16")
            divisor = stored.to(work).unsqueeze(-1)
            live = divisor > 0
            quotient = grouped / torch.where(live, divisor, torch.ones_like(divisor))
            q = torch.where(live, quotient.round().clamp(lowest, levels), torch.zeros_like(quotient))
            codes[rows] = q.reshape(block.shape[0], padded).to(code_dtype)
            scales[rows] = stored
    return codes, scales


def _check_code_source(codes, scales, lo, hi, name):
    _raise_first((
        (lambda: codes.device.type != "cpu" or scales.device.type != "cpu", ValueError,
         "from_codes is an explicit CPU preparation operation"),
        (lambda: codes.dtype not in _SIGNED, ValueError, "codes must contain signed integers"),
        (lambda: codes.ndim != 2 or min(codes.shape) <= 0, ValueError, "codes must be a nonempty [N, K] matrix"),
        (lambda: scales.dtype != torch.float16 or tuple(scales.shape) != (codes.shape[0], (codes.shape[1] + 63) // 64),
         ValueError, "scales must be float16 [N, ceil(K/64)]"),
        (lambda: bool(((codes < lo) | (codes > hi)).any()), ValueError, f"{name} codes must be in [{lo}, {hi}]"),
        (lambda: not bool(torch.isfinite(scales).all()), ValueError, "scales must be finite"),
    ))


def _pad_columns(codes, padded):
    out = torch.zeros((codes.shape[0], padded), dtype=torch.int16)
    out[:, : codes.shape[1]] = codes.to(torch.int16)
    return out


def _pad_groups(scales, groups):
    out = torch.zeros((scales.shape[0], groups), dtype=torch.float16)
    out[:, : scales.shape[1]] = scales
    return out


# ---------------------------------------------------------------- descriptors


@dataclass(frozen=True)
class DenseWeight:
    """A contiguous floating [out_features, in_features] matrix (weights.py:8-51)."""

    data: torch.Tensor

    format = "dense"

    def __post_init__(self):
        self.validate()

    @property
    def in_features(self):
        return self.data.shape[1]

    @property
    def out_features(self):
        return self.data.shape[0]

    @property
    def nbytes(self):
        return self.data.numel() * self.data.element_size()

    def validate(self):
        d = self.data
        _raise_first((
            (lambda: not isinstance(d, torch.Tensor), TypeError, "DenseWeight requires a tensor"),
            (lambda: d.ndim != 2 or not all(_int32_extent(e) for e in d.shape), ValueError,
             "DenseWeight requires a nonempty int32 [N, K] matrix"),
            (lambda: d.dtype not in _FLOATS, ValueError, "DenseWeight requires floating-point storage"),
            (lambda: d.device.type not in ("cpu", "cuda") or not d.is_contiguous(), ValueError,
             "DenseWeight requires contiguous CPU/CUDA storage"),
        ))


class _NibbleRowSplit:
    """Shared geometry checks of the group-64 nibble codecs (Q4, Q5).

    Subclasses set ``_extra_planes`` (field, Kp divisor of its row bytes,
    shape message) for every uint8 plane besides the codes, and the messages
    that name their dtype and device violations.
    """

    group_size = 64
    layout = "row_split_k128_v1"
    _tag = ""
    _extra_planes = ()  # (field, bytes per row = Kp // divisor, shape message)

    @property
    def out_features(self) -> int:
        return self.codes.shape[0]

    @property
    def padded_k(self) -> int:
        return _padded(self.in_features)

    def _tensors(self):
        return (self.codes,) + tuple(getattr(self, f) for f, _, _ in self._extra_planes) + (self.scales,)

    def validate(self) -> None:
        tag, kp = self._tag, lambda: self.padded_k
        extras = [(getattr(self, f), div, msg) for f, div, msg in self._extra_planes]
        tensors = self._tensors()
        rules = [
            (lambda: not _int32_extent(self.in_features), ValueError, "in_features must be a positive int32"),
            (lambda: kp() >= _INT32, ValueError, "padded K must fit int32"),
            (lambda: self.codes.ndim != 2 or not _int32_extent(self.codes.shape[0]), ValueError,
             "codes must be a nonempty [N, padded_K/2] matrix"),
            (lambda: any(t.dtype != torch.uint8 for t in tensors[:-1]) or self.scales.dtype != torch.float16,
             ValueError, self._dtype_message),
            (lambda: self.codes.shape[1] != kp() // 2, ValueError, "codes width must match K padded to 128"),
        ]
        rules += [(lambda t=t, div=div: tuple(t.shape) != (self.out_features, kp() // div), ValueError, msg)
                  for t, div, msg in extras]
        rules += [
            (lambda: tuple(self.scales.shape) != (self.out_features, kp() // 64), ValueError,
             "scales shape must be [N, padded_K/64]"),
            (lambda: not all(t.is_contiguous() for t in tensors), ValueError, f"{tag} planes must be contiguous"),
            (lambda: len({t.device for t in tensors}) != 1, ValueError, self._device_message),
            (lambda: self.codes.device.type not in ("cpu", "cuda"), ValueError,
             f"{tag} planes require CPU or CUDA storage"),
            (lambda: self.scales.data_ptr() % 2 != 0, ValueError, "FP16 scales must be aligned"),
        ]
        _raise_first(rules)


@dataclass(frozen=True)
class Q4RowSplitWeight(_NibbleRowSplit):
    """Signed two's-complement nibbles, group-64 fp16 scales, K padded to 128.

    codes is uint8 [N, padded_K/2] with weight 2j in the low nibble; scales is
    float16 [N, padded_K/64]; values are q * scale with q in [-8, 7].
    """

    codes: torch.Tensor
    scales: torch.Tensor
    in_features: int

    format = "q4_g64_fp16"
    _tag = "Q4"
    _dtype_message = "Q4 requires uint8 codes and float16 scales"
    _device_message = "codes and scales must be on the same device"

    def __post_init__(self):
        self.validate()

    @property
    def nbytes(self) -> int:
        return self.codes.numel() + 2 * self.scales.numel()

    @classmethod
    def from_codes(cls, codes: torch.Tensor, scales: torch.Tensor):
        """Packs CPU integer codes in [-8, 7] exactly (weights.py:108-130); no float quantization."""
        _check_code_source(codes, scales, -8, 7, "Q4")
        k = codes.shape[1]
        padded = _padded(k)
        return cls(_nibbles(_pad_columns(codes, padded)), _pad_groups(scales, padded // 64), k)

    @classmethod
    def from_payload(cls, payload: torch.Tensor, *, out_features: int, in_features: int):
        """Views one encoded payload: codes, then the fp16 scale plane at the next 256-byte boundary."""
        _raise_first((
            (lambda: not _int32_extent(out_features), ValueError, "out_features must be a positive int32"),
            (lambda: not _int32_extent(in_features), ValueError, "in_features must be a positive int32"),
            (lambda: payload.dtype != torch.uint8 or payload.ndim != 1, ValueError,
             "payload must be a contiguous uint8 vector"),
            (lambda: not payload.is_contiguous() or payload.data_ptr() % 2 != 0, ValueError,
             "payload must be contiguous and FP16 aligned"),
        ))
        padded = _padded(in_features)
        code_bytes = out_features * padded // 2
        scale_at = -(-code_bytes // 256) * 256
        if payload.numel() != scale_at + out_features * (padded // 64) * 2:
            raise ValueError("payload byte count does not match the Q4 layout")
        codes = payload[:code_bytes].view(out_features, padded // 2)
        scales = payload[scale_at:].view(torch.float16).view(out_features, padded // 64)
        return cls(codes, scales, in_features)

    def dequantize_reference(self) -> torch.Tensor:
        """CPU FP64 values q * scale (diagnostic; never used by device execution)."""
        self.validate()
        if self.codes.device.type != "cpu":
            raise ValueError("reference decoding requires explicit CPU weights")
        return _group_values(_signed(_unnibble(self.codes), 4), self.scales, 64, self.in_features)


@dataclass(frozen=True)
class Q5RowSplitWeight(_NibbleRowSplit):
    """Signed 5-bit codes, group-64 fp16 scales, K padded to 128 (weights.py:175-336).

    codes is uint8 [N, padded_K/2] with the low four bits of weight 2j in the
    low nibble of byte j; high is uint8 [N, padded_K/8] with the fifth bit of
    column c at bit c % 8 of byte c / 8 (inside each K64 group lane L reads
    byte L//8, bit L%8); scales is float16 [N, padded_K/64]. Values are
    q * scale with q in [-16, 15], no zero point.
    """

    codes: torch.Tensor
    high: torch.Tensor
    scales: torch.Tensor
    in_features: int

    format = "q5_g64_fp16"
    _tag = "Q5"
    _dtype_message = "Q5 requires uint8 codes/high and float16 scales"
    _device_message = "Q5 planes must share one device"
    _extra_planes = (("high", 8, "high plane shape must be [N, padded_K/8]"),)

    def __post_init__(self):
        self.validate()

    @property
    def nbytes(self) -> int:
        return self.codes.numel() + self.high.numel() + 2 * self.scales.numel()

    @classmethod
    def from_codes(cls, codes: torch.Tensor, scales: torch.Tensor):
        """Packs CPU integer codes in [-16, 15] exactly; no float quantization."""
        _check_code_source(codes, scales, -16, 15, "Q5")
        k = codes.shape[1]
        padded = _padded(k)
        unsigned = _pad_columns(codes, padded) & 31
        return cls(_nibbles(unsigned), _bitplane(unsigned >> 4), _pad_groups(scales, padded // 64), k)

    @classmethod
    def from_dense(cls, source, *, rows_per_chunk=256):
        """Nearest-even RTN with the stored fp16 scale fp16(max|group|/15), codes in
        [-16, 15], over K64 groups, chunked by rows; the source is not modified."""
        codes, scales = _rtn_codes(source, group=64, levels=15, lowest=-16, name="Q5", rows_per_chunk=rows_per_chunk,
                                   code_dtype=torch.int16)
        k = source.shape[1]
        return cls.from_codes(codes[:, :k], scales[:, : (k + 63) // 64])

    def dequantize_reference(self) -> torch.Tensor:
        """CPU FP64 values q * scale (diagnostic; never used by device execution)."""
        self.validate()
        if self.codes.device.type != "cpu":
            raise ValueError("reference decoding requires explicit CPU weights")
        unsigned = _unnibble(self.codes) | (_unbitplane(self.high) << 4)
        return _group_values(_signed(unsigned, 5), self.scales, 64, self.in_features)


@dataclass(frozen=True)
class Q8RowSplitWeight:
    """Signed Q8 codes in [-127, 127] with group-32 fp16 scales, K padded to 128."""

    codes: torch.Tensor
    scales: torch.Tensor
    in_features: int

    format = "q8_g32_fp16"
    layout = "row_split_k128_v1"
    group_size = 32

    def __post_init__(self):
        self.validate()

    @property
    def out_features(self):
        return self.codes.shape[0]

    @property
    def padded_k(self):
        return _padded(self.in_features)

    @property
    def nbytes(self):
        return self.codes.numel() + 2 * self.scales.numel()

    def validate(self):
        c, s = self.codes, self.scales
        _raise_first((
            (lambda: not _int32_extent(self.in_features) or self.padded_k >= _INT32, ValueError,
             "Q8 in_features/padded K must be positive int32"),
            (lambda: not (isinstance(c, torch.Tensor) and isinstance(s, torch.Tensor)), TypeError,
             "Q8 requires code and scale tensors"),
            (lambda: c.ndim != 2 or not _int32_extent(c.shape[0]), ValueError, "Q8 codes require nonempty [N,padded_K]"),
            (lambda: c.shape[1] != self.padded_k or c.dtype != torch.int8, ValueError,
             "Q8 codes require int8 [N,padded_K]"),
            (lambda: tuple(s.shape) != (self.out_features, self.padded_k // 32) or s.dtype != torch.float16,
             ValueError, "Q8 scales require float16 [N,padded_K/32]"),
            (lambda: c.device != s.device or c.device.type not in ("cpu", "cuda"), ValueError,
             "Q8 planes require the same CPU/CUDA device"),
            (lambda: not (c.is_contiguous() and s.is_contiguous()), ValueError, "Q8 planes must be contiguous"),
        ))

    @classmethod
    def from_dense(cls, source, *, rows_per_chunk=256):
        """Nearest-even quantization with the stored fp16 scale (weights.py:398-439).

        Per 32-column group: scale = fp16(max|x| / 127) computed in the working
        precision (f32, or f64 for f64 sources); code = clamp(round_half_even(
        x / scale), -127, 127), or 0 where the stored scale is 0. Non-finite
        sources and scales that overflow fp16 are rejected.
        """
        codes, scales = _rtn_codes(source, group=32, levels=127, lowest=-127, name="Q8", rows_per_chunk=rows_per_chunk,
                                   code_dtype=torch.int8)
        return cls(codes, scales, source.shape[1])

    def dequantize_reference(self):
        """CPU FP64 values code * scale, rejecting invalid planes (weights.py:441-454)."""
        self.validate()
        if self.codes.device.type != "cpu":
            raise ValueError("Reference decoding requires explicit CPU planes")
        valid = (not bool((self.codes == -128).any()) and bool(torch.isfinite(self.scales).all())
                 and not bool((self.scales < 0).any()))
        if not valid:
            raise ValueError("Invalid Q8 codes/scales")
        return _group_values(self.codes, self.scales, 32, self.in_features)


# ---------------------------------------------------------------- K64 model encoders


def rtn_k64(weight, *, levels, lowest, tag, max_elements):
    """Symmetric round-to-nearest-even over K64 groups for the model codecs (Q4, Q5).

    Per group: the fp16 scale is rounded first, s = fp16(max(max|w| / levels,
    2^-24)) in fp32; codes = clamp(round_half_even(w / f32(s)), lowest,
    levels) (a code past `levels` can only come from the scale's rounding).
    The source must be a nonempty finite CPU fp16/bf16/fp32 matrix within
    `max_elements`; rejects scales that overflow fp16 and decoded weights
    fp16(q * s) that overflow. Returns signed codes [N, K] and scales
    [N, ceil(K/64)], ready for ``from_codes``.
    """
    ok = (isinstance(weight, torch.Tensor) and weight.device.type == "cpu" and weight.ndim == 2
          and weight.dtype in (torch.float16, torch.bfloat16, torch.float32) and min(weight.shape) >= 1)
    if not ok:
        raise ValueError("Explicit nonempty CPU floating weight required")
    if type(max_elements) is not int or not 0 < max_elements or weight.numel() > max_elements:
        raise ValueError(f"{tag} quantization exceeds explicit element budget")
    source = weight.float()
    if not bool(torch.isfinite(source).all()):
        raise ValueError("Finite source weights required")
    n, k = weight.shape
    groups = torch.nn.functional.pad(source, (0, _padded(k) - k)).view(n, -1, 64)
    scales = torch.clamp_min(groups.abs().amax(-1) / levels, 2.0**-24).half()
    if not bool(torch.isfinite(scales).all()):
        raise ValueError("Source scale overflows FP16")
    step = scales.float()[..., None]
    codes = torch.clamp((groups / step).round(), lowest, levels).to(torch.int8)
    if not bool(torch.isfinite((codes.float() * step).half()).all()):
        raise ValueError("Quantized weight overflows FP16 execution")
    return codes.view(n, -1)[:, :k], scales[:, : (k + 63) // 64]


def decode_k64_fp16(weight, bits):
    """fp16(q * scale) over columns [0, K) of a Q4 (bits 4) or Q5 (bits 5) descriptor."""
    weight.validate()
    unsigned = _unnibble(weight.codes)
    if bits == 5:
        unsigned = unsigned | (_unbitplane(weight.high) << 4)
    q = _signed(unsigned, bits).float().view(weight.out_features, -1, 64)
    return (q * weight.scales.float()[..., None]).view(weight.out_features, -1)[:, : weight.in_features].half()
