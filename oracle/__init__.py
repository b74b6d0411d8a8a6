"""CPU oracle for the quantized-linear path. TEST INFRASTRUCTURE ONLY.

Imported by tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s
cpu_baseline leg, always as the checker or the timed CPU baseline and never
as the product path (venturi_amd never imports this package).

Two layers:

* ``liboracle.so`` (oracle.c, built by ``make -C oracle``): the reference's
  device arithmetic restated in C, in the reference's association order.
* numpy restatements of the codecs (pack/unpack/RTN) and of the MoE combine.

Each function cites the reference file:line it restates (paths relative to
/root/reference/src/venturi/). The tests that pin each function against the
reference's known answers and against closed forms are tests/test_golden.py,
tests/test_weights.py, tests/test_oracle_q4_moe.py, tests/test_q5_codec.py and
tests/test_silu_oracle.py (SwiGLU / SiLU against FP64 over every finite fp16
input); functions that nothing pins are marked "parity unpinned" below.
"""

import ctypes as C
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
LIBRARY = _HERE / "liboracle.so"

_lib = None


def lib():
    """Loads liboracle.so (build it with ``make -C oracle``)."""
    global _lib
    if _lib is None:
        if not LIBRARY.is_file():
            raise FileNotFoundError(f"{LIBRARY} is not built; run make -C oracle")
        handle = C.CDLL(str(LIBRARY))
        P, I, F = C.c_void_p, C.c_int, C.c_float
        handle.oracle_f32_to_f16.argtypes, handle.oracle_f32_to_f16.restype = [F], C.c_uint16
        handle.oracle_f16_to_f32.argtypes, handle.oracle_f16_to_f32.restype = [C.c_uint16], F
        handle.oracle_q8_linear.argtypes = [P, I, P, P, P] + [I] * 4
        handle.oracle_a8_quantize.argtypes = [P, I, I, I, P, P]
        handle.oracle_a8_linear.argtypes = [P] * 5 + [I] * 5
        handle.oracle_a8_group_dots.argtypes = [P] * 3 + [I] * 4
        handle.oracle_rms.argtypes = [P, I, P, P, I, I, F, P]
        handle.oracle_rms_a8.argtypes = [P, P, I, I, F, I, P, P, P, P]
        handle.oracle_q4_linear.argtypes = [P] * 4 + [I] * 4
        handle.oracle_q4_decode.argtypes = [P] * 3 + [I] * 3
        handle.oracle_q4_generic.argtypes = [P] * 4 + [I] * 5
        handle.oracle_q4_fused.argtypes = [P] * 4 + [I] * 4
        handle.oracle_row_decode.argtypes = [P] * 5 + [I] * 4
        handle.oracle_q5_linear.argtypes = [P] * 5 + [I] * 4
        _lib = handle
    return _lib


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p)


def _u16(a):
    """View fp16/bf16 storage (numpy float16 or uint16) as contiguous uint16."""
    a = np.ascontiguousarray(a)
    return a.view(np.uint16) if a.dtype == np.float16 else a.astype(np.uint16, copy=False)


# ---------------------------------------------------------------- Q8 codec


def q8_pack(source):
    """Q8RowSplitWeight.from_dense (ops/weights.py:398-439) in numpy.

    source: float32 (or float64) [n, k]. Returns (codes int8 [n, Kp], scales
    float16 [n, Kp/32]). Raises ValueError for non-finite input or fp16 scale
    overflow, as the reference does.
    """
    source = np.asarray(source)
    work = np.float64 if source.dtype == np.float64 else np.float32
    n, k = source.shape
    padded = (k + 127) // 128 * 128
    block = np.zeros((n, padded), dtype=work)
    block[:, :k] = source
    if not np.isfinite(block).all():
        raise ValueError("Q8 source must be finite")
    groups = block.reshape(n, -1, 32)
    amax = np.abs(groups).max(-1)
    with np.errstate(over="ignore"):
        stored = (amax / work(127)).astype(np.float16)
    if not np.isfinite(stored).all():
        raise ValueError("Q8 group scale overflows FP16")
    divisor = stored.astype(work)[:, :, None]
    safe = np.where(divisor > 0, divisor, work(1))
    q = np.where(divisor > 0, np.clip(np.rint(groups / safe), -127, 127), 0)
    return q.astype(np.int8).reshape(n, padded), stored


def q8_unpack(codes, scales, k):
    """FP64 value code*scale (ops/weights.py:441-454), columns [0, k)."""
    return (codes.astype(np.float64) * np.repeat(scales.astype(np.float64), 32, axis=1))[:, :k]


# ---------------------------------------------------------------- Q4 codec


def q4_pack_codes(codes, scales):
    """Q4RowSplitWeight.from_codes (ops/weights.py:108-130): exact nibble packing."""
    codes = np.asarray(codes)
    n, k = codes.shape
    if ((codes < -8) | (codes > 7)).any():
        raise ValueError("Q4 codes must be in [-8, 7]")
    padded = (k + 127) // 128 * 128
    nib = np.zeros((n, padded), dtype=np.uint8)
    nib[:, :k] = (codes.astype(np.int16) & 15).astype(np.uint8)
    packed = nib[:, 0::2] | (nib[:, 1::2] << 4)
    plane = np.zeros((n, padded // 64), dtype=np.float16)
    plane[:, : scales.shape[1]] = scales
    return packed, plane


def q4_unpack_signed(packed, k):
    """Signed codes [n, k] from packed nibbles (low nibble = even column)."""
    lo = (packed & 15).astype(np.int16)
    hi = (packed >> 4).astype(np.int16)
    values = np.stack((lo, hi), -1).reshape(packed.shape[0], -1)[:, :k]
    return np.where(values < 8, values, values - 16)


def q4_rtn(weight):
    """quantize_q4_rtn (models/flash_next/flash_next_q4.py:26-52) in numpy float32.

    Returns (signed codes int8 [n, k], scales float16 [n, ceil(k/64)]).
    """
    value = np.asarray(weight, dtype=np.float32)
    rows, cols = value.shape
    padded = (cols + 127) // 128 * 128
    blocks = np.zeros((rows, padded), dtype=np.float32)
    blocks[:, :cols] = value
    blocks = blocks.reshape(rows, padded // 64, 64)
    scales = np.maximum(np.abs(blocks).max(-1) / np.float32(7), np.float32(2.0**-24)).astype(np.float16)
    codes = np.clip(np.rint(blocks / scales.astype(np.float32)[:, :, None]), -7, 7).astype(np.int8)
    return codes.reshape(rows, padded)[:, :cols], scales[:, : (cols + 63) // 64]


def q4_decode_fp16(packed, scales, k):
    """fp16(q * scale) (flash_next_q4.py:55-62; flash_next_q4.cu:7-14)."""
    signed = q4_unpack_signed(packed, packed.shape[1] * 2).astype(np.float32)
    values = signed.reshape(packed.shape[0], -1, 64) * scales.astype(np.float32)[:, :, None]
    return values.reshape(packed.shape[0], -1)[:, :k].astype(np.float16)


def pack_high(upper, hb):
    """High plane of a Q5/Q6 row codec (weights.py:175-190, weight_dequant.cuh:1-9).

    ``upper`` [n, padded] holds each column's bits above the low nibble
    (0 <= v < 2**hb); column c's bits go to bits [c*hb, c*hb + hb) of the
    row's LSB-first bit stream. Returns uint8 [n, padded*hb/8].
    """
    upper = np.asarray(upper, dtype=np.int64)
    n, padded = upper.shape
    bits = ((upper[:, :, None] >> np.arange(hb)) & 1).reshape(n, padded * hb)
    return (bits.reshape(n, -1, 8) << np.arange(8)).sum(-1).astype(np.uint8)


def pack_row_codec(codes, scales, bits):
    """Signed codes [n, padded] in the bits-wide range -> (codes, high) planes."""
    codes = np.asarray(codes, dtype=np.int64)
    u = codes & ((1 << bits) - 1)
    low = (u & 15).astype(np.uint8)
    packed = low[:, 0::2] | (low[:, 1::2] << 4)
    high = pack_high(u >> 4, bits - 4) if bits > 4 else np.zeros((codes.shape[0], 0), np.uint8)
    return packed.astype(np.uint8), high, np.asarray(scales, dtype=np.float16)


def row_decode(codes, high, scales, k, bits, ids=None):
    """venturi_row_dequant_rows / _indexed (weight_dequant.cuh:16-67): fp16 bits [len(ids), k]."""
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    high = np.ascontiguousarray(high, dtype=np.uint8) if bits > 4 else np.zeros(1, np.uint8)
    n, padded = codes.shape[0], codes.shape[1] * 2
    ids = np.arange(n, dtype=np.int64) if ids is None else np.ascontiguousarray(ids, dtype=np.int64)
    out = np.zeros((ids.size, k), dtype=np.uint16)
    lib().oracle_row_decode(_ptr(codes), _ptr(high), _ptr(_u16(scales)), _ptr(ids), _ptr(out), ids.size, k, padded,
                            bits)
    return out


# -------------------------------------------------- device-order restatements


def q8_linear(x, codes, scales, k, dtype=0):
    """venturi_q8_head_run canonical bytes (ops/csrc/blocks.cu:306-321).

    x: uint16 (fp16 dtype 0 / bf16 dtype 1) [tokens, k]; returns uint16 [tokens, n].
    """
    xs = _u16(x)
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    sc = _u16(scales)
    tokens, n, padded = xs.shape[0], codes.shape[0], codes.shape[1]
    out = np.zeros((tokens, n), dtype=np.uint16)
    lib().oracle_q8_linear(_ptr(xs), dtype, _ptr(codes), _ptr(sc), _ptr(out), tokens, n, k, padded)
    return out


def a8_quantize(x, passes):
    """vdq::quantize (ops/csrc/q8_dp4a.cuh:15-34): (codes int8 [P,T,G,32], scales f32 [P,T,G])."""
    xs = _u16(x)
    tokens, k = xs.shape
    groups = (k + 31) // 32
    codes = np.zeros((passes, tokens, groups, 32), dtype=np.int8)
    scales = np.zeros((passes, tokens, groups), dtype=np.float32)
    lib().oracle_a8_quantize(_ptr(xs), tokens, k, passes, _ptr(codes), _ptr(scales))
    return codes, scales


def a8_workspace(codes, scales):
    """The reference workspace bytes: all codes, then all scales."""
    return np.concatenate([codes.reshape(-1).view(np.uint8), scales.reshape(-1).view(np.uint8)])


def a8_linear(acodes, ascales, codes, wscales, k):
    """vdq::dot (ops/csrc/q8_dp4a.cuh:36-70): fp16 bits [tokens, n]."""
    acodes = np.ascontiguousarray(acodes, dtype=np.int8)
    ascales = np.ascontiguousarray(ascales, dtype=np.float32)
    passes, tokens = acodes.shape[0], acodes.shape[1]
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    n, padded = codes.shape
    out = np.zeros((tokens, n), dtype=np.uint16)
    lib().oracle_a8_linear(
        _ptr(acodes), _ptr(ascales), _ptr(codes), _ptr(_u16(wscales)), _ptr(out), tokens, n, k, padded, passes
    )
    return out


def a8_group_dots(acodes, codes, k):
    """Exact int32 per-group dots of pass 0: [tokens, n, groups]."""
    acodes = np.ascontiguousarray(acodes[0], dtype=np.int8)
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    tokens, groups = acodes.shape[0], acodes.shape[1]
    n, padded = codes.shape
    dots = np.zeros((tokens, n, groups), dtype=np.int32)
    lib().oracle_a8_group_dots(_ptr(acodes), _ptr(codes), _ptr(dots), tokens, n, k, padded)
    return dots


def rms(x, weight, epsilon, dtype=0):
    """rms_norm (ops/csrc/blocks.cu:31-54) with 1/sqrt in place of rsqrtf.

    dtype 0/1: x is uint16 fp16/bf16 bits; dtype 2: float32.
    """
    w = np.ascontiguousarray(weight, dtype=np.float32)
    if dtype == 2:
        xs = np.ascontiguousarray(x, dtype=np.float32)
        out = np.zeros_like(xs)
    else:
        xs = _u16(x)
        out = np.zeros_like(xs)
    tokens, k = xs.shape
    buffer = np.zeros(k, dtype=np.float32)
    lib().oracle_rms(_ptr(xs), dtype, _ptr(w), _ptr(out), tokens, k, epsilon, _ptr(buffer))
    return out


def rms_a8(x, weight, epsilon, passes):
    """RMSNorm -> fp16 -> A8 (ops/csrc/q8_rms_producer.cuh:8-53, any pass count).

    Returns (codes [P,T,G,32], scales [P,T,G], fp16 bits of the normalised rows).
    """
    xs = _u16(x)
    tokens, k = xs.shape
    groups = (k + 31) // 32
    w = np.ascontiguousarray(weight, dtype=np.float32)
    codes = np.zeros((passes, tokens, groups, 32), dtype=np.int8)
    scales = np.zeros((passes, tokens, groups), dtype=np.float32)
    inter = np.zeros((tokens, k), dtype=np.uint16)
    buffer = np.zeros(k, dtype=np.float32)
    lib().oracle_rms_a8(_ptr(xs), _ptr(w), tokens, k, epsilon, passes, _ptr(codes), _ptr(scales), _ptr(inter),
                        _ptr(buffer))
    return codes, scales, inter


def q4_linear(x, packed, scales, k):
    """q4_linear (ops/csrc/flash_next_q4.cu:23-34): fp16 bits [tokens, rows]."""
    xs = _u16(x)
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    tokens, rows, padded = xs.shape[0], packed.shape[0], packed.shape[1] * 2
    out = np.zeros((tokens, rows), dtype=np.uint16)
    lib().oracle_q4_linear(_ptr(xs), _ptr(packed), _ptr(_u16(scales)), _ptr(out), tokens, rows, k, padded)
    return out


def q5_linear(x, codes, high, scales, k):
    """q5_linear (ops/csrc/flash_next_q5.cu:26-38): fp16 bits [tokens, rows]."""
    xs = _u16(x)
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    high = np.ascontiguousarray(high, dtype=np.uint8)
    tokens, rows, padded = xs.shape[0], codes.shape[0], codes.shape[1] * 2
    out = np.zeros((tokens, rows), dtype=np.uint16)
    lib().oracle_q5_linear(_ptr(xs), _ptr(codes), _ptr(high), _ptr(_u16(scales)), _ptr(out), tokens, rows, k, padded)
    return out


def q4_generic(x, packed, scales, k, dtype=0):
    """q4_generic (ops/csrc/q4_linear.cu:21-56): fp16/bf16 bits [tokens, n]."""
    xs = _u16(x)
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    tokens, n, padded = xs.shape[0], packed.shape[0], packed.shape[1] * 2
    out = np.zeros((tokens, n), dtype=np.uint16)
    lib().oracle_q4_generic(_ptr(xs), _ptr(packed), _ptr(_u16(scales)), _ptr(out), n, k, padded, tokens, dtype)
    return out


def q4_fused(x, packed, scales, k):
    """q4_fused_run_kernel (ops/csrc/q4_fused.cuh:10-89): fp16 bits [tokens, rows]."""
    xs = _u16(x)
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    tokens, rows, padded = xs.shape[0], packed.shape[0], packed.shape[1] * 2
    out = np.zeros((tokens, rows), dtype=np.uint16)
    lib().oracle_q4_fused(_ptr(xs), _ptr(packed), _ptr(_u16(scales)), _ptr(out), tokens, rows, k, padded)
    return out


def q4_decode(packed, scales, k):
    """q4_decode (ops/csrc/flash_next_q4.cu:16-21) through the C restatement: fp16 bits [rows, k]."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    rows, padded = packed.shape[0], packed.shape[1] * 2
    out = np.zeros((rows, k), dtype=np.uint16)
    lib().oracle_q4_decode(_ptr(packed), _ptr(_u16(scales)), _ptr(out), rows, k, padded)
    return out


def f32_to_f16_bits(values):
    """Element-wise RNE fp32 -> fp16 through the oracle's own converter."""
    f = lib().oracle_f32_to_f16
    flat = np.asarray(values, dtype=np.float32).reshape(-1)
    return np.array([f(float(v)) for v in flat], dtype=np.uint16).reshape(np.shape(values))


def swiglu(a, b):
    """blocks.cu:56-70 SwiGLU: cast((x * sigmoid(x)) * y), fp32 math, stable logistic; fp16 bits in/out.

    numpy's float32 exp stands in for the device exp. Pinned against FP64
    x * y / (1 + e^-x) rounded once to fp16 (tests/test_silu_oracle.py): equal
    away from rounding midpoints, within one ulp everywhere.
    """
    x = np.asarray(a, np.float16).astype(np.float32)
    y = np.asarray(b, np.float16).astype(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):  # the branch not taken may overflow to inf / inf
        pos = np.float32(1) / (np.float32(1) + np.exp(-x))
        neg = np.exp(x) / (np.float32(1) + np.exp(x))
        sig = np.where(x >= 0, pos, neg).astype(np.float32)
        return ((x * sig).astype(np.float32) * y).astype(np.float16)  # past 65504 -> inf, as the device cast
