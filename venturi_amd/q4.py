"""Q4 (q4_g64_fp16) codec helpers and the W4A16 linear plan.

``quantize_q4_rtn`` and ``decode_q4_fp16`` mirror the reference's expert codec
(models/flash_next/flash_next_q4.py:26-62): fp16 scale = fp16(max|w|/7)
floored at 2^-24, codes = clamp(round_half_even(w / scale), -7, 7), and the
W4A16 weight value fp16(q * scale).
"""

from dataclasses import dataclass
from functools import cached_property

import torch

from .operands import DTYPE_CODES, admit, disjoint, extents, stream_of
from .plugin import CodecEntry, RowCodecOperator
from .weights import Q4RowSplitWeight, decode_k64_fp16, rtn_k64

# Plan routes of a resident Q4 linear:
#   mfma    W4A16 contract (fp16(q*scale) weights) on fp16 matrix cores, any tokens
#           (below DECODE_TILED_TOKENS over the resident's tiled decode copy);
#   generic the plugin order of q4_linear.cu:21-56 (FP32 weights), fp16/bf16;
#   exact   the expert order of flash_next_q4.cu:23-34 (fp16 weights), fp16, <= 64 tokens;
#   fused   the research order of q4_fused.cuh:10-89 (FP32 weights), fp16;
#   dense   the reference's ChunkedDense path (qwen_runtime.cuh:348-364): rows
#           decoded to fp16(q*scale) in the caller's workspace, then hipBLASLt
#           (fp32 accumulation), fp16, k % 8 == 0 and n % 8 == 0; run(x, out=)
#           without a workspace, as the reference calls a plan, runs the mfma
#           GEMM instead (no workspace, the same contract bound).
# auto: for fp16 activations dense from DENSE_TOKENS tokens (where the library
# GEMM outruns the fused matrix-core kernel despite decoding the weights:
# config-2 shapes at 1024 tokens 0.95-1.44x, at 2048 1.36-1.62x), else mfma;
# generic for bf16.
Q4_ROUTES = ("auto", "mfma", "generic", "exact", "fused", "dense")
DECODE_TILED_TOKENS = 32
DENSE_TOKENS = 1024


def tile_q4(codes, scales):
    """Tiled decode copy of row-major Q4 planes (read by ``venturi_q4_tiled_run``).

    Codes [row block][chunk][lane l = 16q + r][16 bytes]: row r of the 16-row
    block, columns 128c + 32q .. +32 of the chunk (the bytes 16q .. 16q+15 of
    the row-major chunk). Inside each 4-byte word (8 columns c .. c+7) the
    nibbles are stored biased (q + 8) and reordered: nibble j holds column
    c + 2j, nibble 4 + j column c + 2j + 1, the order in which the kernel's
    mask-and-or dequant yields natural column order. Scales [row block][chunk]
    [r][2] fp16: the chunk's two groups. Rows past n are zero.
    """
    n, row_bytes = codes.shape
    chunks = row_bytes // 64
    blocks = (n + 15) // 16
    nib = torch.stack((codes & 15, codes >> 4), -1).reshape(n, row_bytes // 4, 8) ^ 8  # biased, column order
    nib = nib[:, :, [0, 2, 4, 6, 1, 3, 5, 7]].reshape(n, row_bytes, 2)
    packed = nib[..., 0] | (nib[..., 1] << 4)
    c = torch.zeros((blocks * 16, row_bytes), dtype=torch.uint8, device=codes.device)
    s = torch.zeros((blocks * 16, chunks * 2), dtype=torch.float16, device=codes.device)
    c[:n] = packed
    s[:n] = scales
    tc = c.view(blocks, 16, chunks, 4, 16).permute(0, 2, 3, 1, 4).contiguous()
    ts = s.view(blocks, 16, chunks, 2).permute(0, 2, 1, 3).contiguous()
    return tc, ts


def quantize_q4_rtn(weight, *, max_elements=16 * 2**20):
    """CPU RTN for the model's Q4 experts (flash_next_q4.py:26-52): per K64 group the fp16
    scale fp16(max(max|w| / 7, 2^-24)) is rounded first, then q = RNE(w / scale) in [-7, 7]
    (the -8 code is never produced); returns a ``Q4RowSplitWeight``."""
    codes, scales = rtn_k64(weight, levels=7, lowest=-7, tag="Q4", max_elements=max_elements)
    return Q4RowSplitWeight.from_codes(codes, scales)


def decode_q4_fp16(weight):
    """fp16 matrix of fp16(q * scale) values, the W4A16 weights (diagnostic; no retained cache)."""
    return decode_k64_fp16(weight, 4)


def _q4_planes(weight):
    if not isinstance(weight, Q4RowSplitWeight):
        raise TypeError("Q4RowSplitWeight required")
    weight.validate()
    if not bool(torch.isfinite(weight.scales).all()):
        raise ValueError("scales must be finite")


@dataclass(frozen=True)
class ResidentQ4Linear:
    """Owned device Q4 planes shared by many token-shape plans."""

    backend: object
    weight: Q4RowSplitWeight
    dtype: torch.dtype

    @property
    def device(self):
        return self.weight.codes.device

    @property
    def storage_tensors(self):
        return (self.weight.codes, self.weight.scales)

    @cached_property
    def tiled(self):
        """The tiled decode copy (``tile_q4``), built on first use by a decode plan."""
        return tile_q4(self.weight.codes, self.weight.scales)

    @property
    def in_features(self):
        return self.weight.in_features

    @property
    def out_features(self):
        return self.weight.out_features

    def prepare(self, *, tokens, route="auto"):
        extents(tokens, self.out_features)
        if tokens * self.out_features >= 2**31:
            raise ValueError("Q4 output count must fit int32")
        if route not in Q4_ROUTES:
            raise ValueError(f"Q4 route must be one of {Q4_ROUTES}")
        fp16 = self.dtype == torch.float16
        dense_ok = fp16 and self.in_features % 8 == 0 and self.out_features % 8 == 0
        if route == "auto":
            if dense_ok and tokens >= DENSE_TOKENS:
                route = "dense"
            else:
                route = "mfma" if fp16 and self.in_features % 8 == 0 else "generic"
        if route == "dense" and not dense_ok:
            raise ValueError("The dense Q4 route takes FP16 activations, K % 8 == 0 and N % 8 == 0")
        if route == "mfma" and not (fp16 and self.in_features % 8 == 0):
            raise ValueError("The Q4 matrix-core route takes FP16 activations and K % 8 == 0")
        if route == "exact" and not (fp16 and tokens <= 64):
            raise ValueError("The exact expert Q4 route takes FP16 activations and at most 64 tokens")
        if route == "fused" and not (fp16 and tokens <= 65535):
            raise ValueError("The fused Q4 route takes FP16 activations")
        if route == "generic" and tokens > 4 * 65535:
            raise ValueError("The generic Q4 route takes at most 262140 tokens")
        self.backend.validate_device(self.dtype, self.device)
        slots = None
        if route == "mfma" and tokens < DECODE_TILED_TOKENS:
            self.tiled  # built once here, so that run allocates nothing
            lib = self.backend._native
            size = int(lib.venturi_q4_tiled_workspace_bytes(tokens, self.out_features, self.in_features))
            if size:
                # A decode that splits K exchanges its halves through slots the
                # plan owns; every run leaves them idle, so runs of one plan must
                # be ordered (one stream), and concurrent streams prepare a plan each.
                slots = torch.empty(size, dtype=torch.uint8, device=self.device)
                with torch.cuda.device(self.device):
                    self.backend._check(lib.venturi_q4_tiled_workspace_init(slots.data_ptr(), size,
                                                                              stream_of(self.device)))
            # The copy and the slots were written on this stream; a plan may run on another.
            torch.cuda.current_stream(self.device).synchronize()
        workspace = 0
        if route == "dense":
            workspace = int(self.backend._native.venturi_row_dense_workspace_bytes(
                tokens, self.out_features, self.in_features))
            if workspace == 0:
                raise ValueError(self.backend._native.error())
        return Q4LinearPlan(self, tokens, route, slots, workspace)

    def decode(self, *, out, row=0):
        """fp16 rows fp16(q * scale) of [row, row + len(out)) into ``out`` (blocks.cu:1077-1086)."""
        rows = out.shape[0] if isinstance(out, torch.Tensor) and out.ndim == 2 else -1
        if type(row) is not int or row < 0 or rows <= 0 or row + rows > self.out_features:
            raise ValueError("Q4 decode rows must lie inside the matrix")
        admit(out, (rows, self.in_features), torch.float16, self.device, "out")
        disjoint(out, self.storage_tensors)
        w = self.weight
        with torch.cuda.device(self.device):
            self.backend._check(
                self.backend._native.venturi_row_dequant_rows(
                    w.codes.data_ptr(), None, w.scales.data_ptr(), out.data_ptr(), row, rows, w.in_features,
                    w.padded_k, 4, stream_of(self.device),
                )
            )
        return out


@dataclass(frozen=True)
class Q4LinearPlan:
    """out[T, N] = x[T, K] @ W[N, K]^T without bias; caller-owned buffers only."""

    resident: ResidentQ4Linear
    tokens: int
    kernel: str
    slots: object = None  # exchange slots of a decode that splits K (plan-owned)
    workspace_bytes: int = 0  # the dense route's caller-owned shadow and hipBLASLt workspace

    @property
    def route(self):
        return "venturi-q4-" + self.kernel

    @property
    def dtype(self):
        return self.resident.dtype

    @property
    def device(self):
        return self.resident.device

    @property
    def in_features(self):
        return self.resident.in_features

    @property
    def out_features(self):
        return self.resident.out_features

    @property
    def storage_tensors(self):
        r = self.resident
        return r.storage_tensors + (r.tiled if self.kernel == "mfma" and self.tokens < DECODE_TILED_TOKENS else ())

    def run(self, x, *, out, workspace=None):
        r = self.resident
        if self.kernel != "dense" and workspace is not None:
            raise ValueError("Q4 Linear uses no workspace")
        admit(x, (self.tokens, r.in_features), r.dtype, r.device, "x")
        admit(out, (self.tokens, r.out_features), r.dtype, r.device, "out")
        disjoint(out, (x,) + self.storage_tensors)
        kernel = self.kernel
        if kernel == "dense" and workspace is None:
            # The reference's run(x, out=) passes no workspace: the fused
            # matrix-core GEMM, which needs none, serves the call.
            kernel = "mfma"
        if kernel == "dense":
            admit(workspace, (self.workspace_bytes,), torch.uint8, r.device, "workspace")
            if workspace.data_ptr() % 256 or x.data_ptr() % 16 or out.data_ptr() % 16:
                raise ValueError("the dense Q4 route needs a 256-byte aligned workspace and 16-byte aligned x and out")
            disjoint(workspace, (x, out) + self.storage_tensors)
        w, lib, stream = r.weight, r.backend._native, stream_of(r.device)
        args = (x.data_ptr(), w.codes.data_ptr(), w.scales.data_ptr(), out.data_ptr())
        with torch.cuda.device(r.device):
            if kernel == "dense":
                status = lib.venturi_row_dense_run(
                    *args[:2], None, *args[2:], self.tokens, w.out_features, w.in_features, w.padded_k, 4,
                    DTYPE_CODES[r.dtype], workspace.data_ptr(), self.workspace_bytes, stream
                )
            elif kernel == "mfma" and self.tokens < DECODE_TILED_TOKENS:
                tc, ts = r.tiled
                slots = self.slots
                status = lib.venturi_q4_tiled_run(
                    x.data_ptr(), tc.data_ptr(), ts.data_ptr(), out.data_ptr(), self.tokens, w.out_features,
                    w.in_features, w.padded_k, DTYPE_CODES[r.dtype], None if slots is None else slots.data_ptr(),
                    0 if slots is None else slots.numel(), stream
                )
            elif kernel == "mfma":
                status = lib.venturi_q4_gemm_run(
                    *args, self.tokens, w.out_features, w.in_features, w.padded_k, DTYPE_CODES[r.dtype], stream
                )
            elif self.kernel == "generic":
                status = lib.venturi_q4_run(
                    *args, w.out_features, w.in_features, w.padded_k, self.tokens, DTYPE_CODES[r.dtype], 0, stream
                )
                if status < 0:
                    raise RuntimeError(lib.venturi_ada_error().decode("utf-8", "replace"))
            elif self.kernel == "exact":
                code = lib.venturi_q4_linear(*args, self.tokens, w.out_features, w.in_features, w.padded_k, stream)
                if code:
                    raise RuntimeError(f"Q4 GEMV HIP launch failed: {code}")
                status = 0
            else:
                status = lib.venturi_q4_fused_run(
                    *args, self.tokens, w.out_features, w.in_features, w.padded_k, 0, stream
                )
            r.backend._check(status)
        return out


def upload_q4(backend, weight, *, device, dtype):
    """Copies the Q4 planes to the device once (reference ada.py:46-58)."""
    _q4_planes(weight)
    if dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("Q4 activations require float16 or bfloat16")
    target = backend.validate_device(dtype, device)
    with torch.cuda.device(target):
        codes = weight.codes.detach().to(target, copy=True)
        scales = weight.scales.detach().to(target, copy=True)
        torch.cuda.current_stream(target).synchronize()
    return ResidentQ4Linear(backend, Q4RowSplitWeight(codes, scales, weight.in_features), dtype)


# ---------------------------------------------------------------------------
# The reference's stand-alone Q4 operator object, over the same library.


@dataclass(frozen=True)
class PreparedQ4:
    weight: Q4RowSplitWeight
    ready: object


class NativeQ4(RowCodecOperator):
    """Expert Q4 operators of ABI 1 (reference ops/flash_next_q4.py:17-89).

    ``linear`` is the expert GEMV order (fp16(q*scale) weights, lane-strided
    fmaf, 32-lane tree) for 1..64 fp16 tokens; ``decode`` writes the fp16
    matrix. Device qualification is gfx950 instead of SM70.
    """

    entry = CodecEntry("Q4", Q4RowSplitWeight, ("codes", "scales"), "venturi_q4_abi", "venturi_q4_decode",
                       "venturi_q4_linear")
    prepared = PreparedQ4
