"""HIP backend: uploads, shape plans and explicit-buffer execution on gfx950.

Mirrors the reference's prepared-operator layer (venturi.ops.blocks,
blocks.py:27-581): ``ResidentLinear`` / ``ResidentRMSNorm`` records, the same
operand guards (exact shape, dtype and device, contiguity, no aliasing,
inference only), and plans whose ``run`` performs no allocation,
synchronisation or implicit cast, so they can be captured in HIP graphs.
Every kernel is called through the C ABI of libventuri_ops.so.
"""

import ctypes
from dataclasses import dataclass
import math

import torch

from . import native
from .backend import Backend, BackendCapabilities, OperatorSupport, UnsupportedOperationError
from .weights import DenseWeight, Q4RowSplitWeight, Q8RowSplitWeight

_DTYPES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}

Q8_ROUTES = ("auto", "exact", "mfma", "dense")


def _shape(tokens, features):
    if any(type(v) is not int or not 0 < v < 2**31 for v in (tokens, features)):
        raise ValueError("tokens and features must be positive int32 values")
    return (tokens, features)


def _tensor(tensor, shape, dtype, device, name):
    if not isinstance(tensor, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if tensor.shape != shape or tensor.dtype != dtype or tensor.device != device:
        raise ValueError(f"{name} requires shape {shape}, dtype {dtype}, device {device}")
    if not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous; no implicit copy")
    if torch.is_grad_enabled() and tensor.requires_grad:
        raise ValueError("Prepared operators are inference-only")


def _overlaps(a, b):
    """Byte-interval overlap of two contiguous tensors on one device."""
    return a.device == b.device and max(a.data_ptr(), b.data_ptr()) < min(
        a.data_ptr() + a.numel() * a.element_size(), b.data_ptr() + b.numel() * b.element_size()
    )


def _no_overlap(out, operands, *, allow_inplace=False):
    for operand in operands:
        if _overlaps(out, operand) and not (
            allow_inplace
            and out.data_ptr() == operand.data_ptr()
            and out.shape == operand.shape
            and out.dtype == operand.dtype
        ):
            raise ValueError("output/workspace must not alias operand storage")


def _epsilon(value):
    if (
        type(value) not in (float, int)
        or not math.isfinite(value)
        or not torch.finfo(torch.float32).tiny <= value <= torch.finfo(torch.float32).max
        or ctypes.c_float(value).value == 0
    ):
        raise ValueError("epsilon must be finite, positive, and a normal FP32 value")
    return float(value)


def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


@dataclass(frozen=True)
class ResidentLinear:
    """One owned weight upload shared by many shape plans (blocks.py:67-101)."""

    _backend: object
    _payload: object
    storage_tensors: tuple
    dtype: torch.dtype
    device: torch.device
    in_features: int
    out_features: int

    @property
    def storage_nbytes(self):
        return sum(t.numel() * t.element_size() for t in self.storage_tensors)

    def prepare_embedding(self, token_ids):
        from .vocabulary import ResidentQ8Vocabulary

        if isinstance(self._payload, ResidentQ8Vocabulary):
            return self._payload.prepare_embedding(token_ids)
        raise UnsupportedOperationError("Embedding lookup is defined for Q8 weights only")

    def prepare(self, *, tokens, route="auto"):
        _shape(tokens, self.in_features)
        self._backend.validate_device(self.dtype, self.device)
        return self._backend.bind_linear(self, tokens=tokens, route=route)

    def prepare_swiglu(self, *, tokens):
        """Fused gate+up projection and SwiGLU for a Q8 [2 * inter, hidden] weight, gate rows
        first (an extension: the native runtime runs the projection, then SwiGLU). The plan's
        output is [tokens, inter]."""
        from .vocabulary import ResidentQ8Vocabulary

        _shape(tokens, self.in_features)
        if not isinstance(self._payload, ResidentQ8Vocabulary):
            raise UnsupportedOperationError("The fused SwiGLU projection is defined for Q8 weights only")
        return _Q8Linear(self._payload.prepare_swiglu(tokens=tokens))


@dataclass(frozen=True)
class ResidentRMSNorm:
    """One owned fp32 norm vector shared across token-shape plans (blocks.py:128-160)."""

    _backend: object
    _weight: torch.Tensor
    dtype: torch.dtype
    epsilon: float

    @property
    def storage_tensors(self):
        return (self._weight,)

    @property
    def storage_nbytes(self):
        return self._weight.numel() * self._weight.element_size()

    @property
    def device(self):
        return self._weight.device

    @property
    def features(self):
        return self._weight.numel()

    def prepare(self, *, tokens):
        _shape(tokens, self.features)
        self._backend.validate_device(self.dtype, self.device)
        return self._backend.bind_rmsnorm(self, tokens=tokens)


def _capabilities():
    devices = frozenset(("cuda",))
    quant = frozenset((torch.float16, torch.bfloat16))
    operators = [
        OperatorSupport("rmsnorm", devices, frozenset((torch.float16, torch.bfloat16, torch.float32))),
        OperatorSupport("linear", devices, quant, "q8_g32_fp16", "row_split_k128_v1"),
        OperatorSupport("embedding", devices, quant, "q8_g32_fp16", "row_split_k128_v1"),
        OperatorSupport("linear", devices, quant, "q4_g64_fp16", "row_split_k128_v1"),
    ]
    return BackendCapabilities("venturi-ops-gfx950", tuple(operators), reference=False, cuda_graphs=True)


def is_gfx950(device):
    """True when the torch device is an MI355X-class (gfx950) GPU."""
    name = getattr(torch.cuda.get_device_properties(device), "gcnArchName", "")
    return name.split(":")[0] == "gfx950"


class HipBackend(Backend):
    """Explicit gfx950 native library; loading never builds or allocates."""

    name = "venturi-ops-hip"
    execution_kind = "native-hip"
    architecture = native.ARCH_TAG

    def __init__(self, library=None):
        self._native = native.load(library)
        self.library = self._native.path

    @property
    def capabilities(self):
        return _capabilities()

    def _check(self, status):
        return self._native.check(status)

    def validate_device(self, dtype, device):
        if dtype not in _DTYPES:
            raise ValueError("Native blocks require FP16, BF16 or FP32")
        return self.resolve_device(device)

    def resolve_device(self, device):
        target = torch.device(device)
        if target.type != "cuda":
            raise ValueError("HipBackend requires an explicit GPU device")
        with torch.cuda.device(target):
            target = torch.device("cuda", torch.cuda.current_device())
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("Preparation must run outside graph capture")
            if not is_gfx950(target):
                raise ValueError("libventuri_ops.so is built for gfx950 (MI355X) only")
        return target

    def empty(self, shape, *, dtype, device):
        if not isinstance(shape, (list, tuple)) or any(type(d) is not int or not 0 <= d < 2**31 for d in shape):
            raise ValueError("Allocation shape must contain nonnegative int32 extents")
        if not isinstance(dtype, torch.dtype):
            raise TypeError("Allocation requires an explicit torch.dtype")
        target = self.validate_device(dtype, device) if dtype.is_floating_point else self.resolve_device(device)
        return torch.empty(tuple(shape), dtype=dtype, device=target)

    def synchronize(self, device):
        torch.cuda.synchronize(self.resolve_device(device))

    # -- linear ------------------------------------------------------------
    def upload_linear(self, weight, *, dtype, device, residency="row-major"):
        """Owned device copy of a weight. ``residency`` (an extension, Q8 only) keeps the
        row-major planes ("row-major"), or only the matrix-core decode's tiled copy
        ("tiled", or "tiled-paired" for a gate+up matrix run by ``prepare_swiglu``)."""
        if not isinstance(weight, (DenseWeight, Q4RowSplitWeight, Q8RowSplitWeight)):
            raise TypeError("Linear requires explicit DenseWeight, Q4RowSplitWeight or Q8RowSplitWeight")
        weight.validate()
        self.require_linear(weight, dtype=dtype, device=device)
        target = self.validate_device(dtype, device)
        if residency != "row-major" and not isinstance(weight, Q8RowSplitWeight):
            raise ValueError("tiled residency is defined for Q8 weights only")
        if isinstance(weight, Q8RowSplitWeight):
            from .vocabulary import Q8VocabularyWeights

            resident = Q8VocabularyWeights(weight.codes, weight.scales, weight.in_features).upload(
                self, device=target, dtype=dtype, residency=residency
            )
        else:
            from .q4 import upload_q4

            resident = upload_q4(self, weight, device=target, dtype=dtype)
        return ResidentLinear(
            self, resident, resident.storage_tensors, dtype, target, weight.in_features, weight.out_features
        )

    def quantize_q8(self, source):
        """Device Q8 packing with the arithmetic of ``Q8RowSplitWeight.from_dense``.

        ``source`` is a contiguous fp16/bf16/fp32 [N, K] tensor on this
        backend's device; the result is a device-resident ``Q8RowSplitWeight``
        whose bytes equal ``Q8RowSplitWeight.from_dense(source.cpu())``.
        (Extension: the reference quantizes on the CPU only.)
        """
        if not isinstance(source, torch.Tensor) or source.ndim != 2 or not source.is_contiguous():
            raise ValueError("Q8 packing requires a contiguous [N, K] tensor")
        if source.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise ValueError("Device Q8 packing supports fp16/bf16/fp32 sources")
        target = self.resolve_device(source.device)
        n, k = source.shape
        _shape(n, k)
        padded = (k + 127) // 128 * 128
        with torch.cuda.device(target):
            if not bool(torch.isfinite(source).all()):
                raise ValueError("Q8 source must be finite")
            if float(source.abs().amax().float()) / 127 >= 65520:
                raise ValueError("Q8 group scale overflows FP16")
            codes = torch.empty(n, padded, dtype=torch.int8, device=target)
            scales = torch.empty(n, padded // 32, dtype=torch.float16, device=target)
            self._check(
                self._native.venturi_q8_pack_run(
                    source.data_ptr(), codes.data_ptr(), scales.data_ptr(), n, k, padded, _DTYPES[source.dtype],
                    _stream(target),
                )
            )
        return Q8RowSplitWeight(codes, scales, k)

    def quantize_q4(self, source):
        """Device Q4 packing with the arithmetic of ``quantize_q4_rtn``.

        ``source`` is a contiguous fp16/bf16/fp32 [N, K] tensor on this
        backend's device; the result is a device-resident ``Q4RowSplitWeight``
        whose bytes equal ``quantize_q4_rtn(source.cpu())``
        (models/flash_next/flash_next_q4.py:26-52). (Extension: the reference
        quantizes on the CPU only.)
        """
        if not isinstance(source, torch.Tensor) or source.ndim != 2 or not source.is_contiguous():
            raise ValueError("Q4 packing requires a contiguous [N, K] tensor")
        if source.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise ValueError("Device Q4 packing supports fp16/bf16/fp32 sources")
        target = self.resolve_device(source.device)
        n, k = source.shape
        _shape(n, k)
        padded = (k + 127) // 128 * 128
        with torch.cuda.device(target):
            if not bool(torch.isfinite(source).all()):
                raise ValueError("Finite source weights required")
            top = torch.clamp_min(source.abs().amax().float() / 7, 2**-24).half()
            if not bool(torch.isfinite(top)) or not bool(torch.isfinite((top.float() * 7).half())):
                raise ValueError("Source scale overflows FP16")
            codes = torch.empty(n, padded // 2, dtype=torch.uint8, device=target)
            scales = torch.empty(n, padded // 64, dtype=torch.float16, device=target)
            self._check(
                self._native.venturi_q4_pack_run(
                    source.data_ptr(), codes.data_ptr(), scales.data_ptr(), n, k, padded, _DTYPES[source.dtype],
                    _stream(target),
                )
            )
        return Q4RowSplitWeight(codes, scales, k)

    def bind_linear(self, resident, *, tokens, route="auto"):
        _shape(tokens, 1)
        if resident._backend is not self:
            raise ValueError("Resident weight belongs to a different backend instance")
        from .vocabulary import ResidentQ8Vocabulary

        if isinstance(resident._payload, ResidentQ8Vocabulary):
            return _Q8Linear(resident._payload.prepare(tokens=tokens, route=route))
        return resident._payload.prepare(tokens=tokens, route=route)

    def prepare_linear(self, weight, *, tokens, dtype, device):
        _shape(tokens, 1)
        return self.upload_linear(weight, dtype=dtype, device=device).prepare(tokens=tokens)

    # -- rmsnorm -----------------------------------------------------------
    def upload_rmsnorm(self, weight, *, dtype, device, epsilon):
        if not isinstance(weight, torch.Tensor) or weight.ndim != 1 or not weight.is_floating_point():
            raise ValueError("RMSNorm weight must be a floating-point vector")
        _shape(1, weight.numel())
        epsilon = _epsilon(epsilon)
        target = self.validate_device(dtype, device)
        with torch.cuda.device(target):
            owned = weight.detach().to(device=target, dtype=torch.float32, copy=True).contiguous()
            if not bool(torch.isfinite(owned).all()):
                raise ValueError("RMSNorm weight must be finite in FP32")
            torch.cuda.current_stream(target).synchronize()
        return ResidentRMSNorm(self, owned, dtype, epsilon)

    def bind_rmsnorm(self, resident, *, tokens):
        _shape(tokens, 1)
        if resident._backend is not self:
            raise ValueError("Resident weight belongs to a different backend instance")
        return _RMSNorm(self, resident._weight, tokens, resident.dtype, resident.epsilon)

    def prepare_rmsnorm(self, weight, *, tokens, dtype, device, epsilon):
        _shape(tokens, 1)
        return self.upload_rmsnorm(weight, dtype=dtype, device=device, epsilon=epsilon).prepare(tokens=tokens)


@dataclass(frozen=True)
class _Q8Linear:
    """LinearPlan adapter over a Q8 output-head plan (blocks.py:735-768)."""

    plan: object

    @property
    def workspace_bytes(self):
        return self.plan.workspace_bytes

    @property
    def route(self):
        return self.plan.route

    @property
    def tokens(self):
        return self.plan.tokens

    @property
    def dtype(self):
        return self.plan.resident.dtype

    @property
    def device(self):
        return self.plan.resident.device

    @property
    def in_features(self):
        return self.plan.resident.hidden_size

    @property
    def out_features(self):
        return self.plan.out_features

    @property
    def storage_tensors(self):
        return self.plan.storage_tensors

    def run(self, x, *, out, workspace=None):
        if workspace is not None and self.plan.workspace_bytes == 0:
            raise ValueError("Direct Q8 Linear uses no workspace")
        return self.plan.run(x, out=out, workspace=workspace)


@dataclass(frozen=True)
class _RMSNorm:
    """RMSNorm plan (blocks.py:789-823); statistics in the reference's reduction order."""

    _backend: HipBackend
    _weight: torch.Tensor
    tokens: int
    dtype: torch.dtype
    epsilon: float
    workspace_bytes = 0

    @property
    def storage_tensors(self):
        return (self._weight,)

    @property
    def device(self):
        return self._weight.device

    @property
    def features(self):
        return self._weight.numel()

    def run(self, x, *, out):
        shape = (self.tokens, self.features)
        _tensor(x, shape, self.dtype, self.device, "x")
        _tensor(out, shape, self.dtype, self.device, "out")
        _no_overlap(out, (x, self._weight))
        with torch.cuda.device(self.device):
            self._backend._check(
                self._backend._native.venturi_rms_run(
                    x.data_ptr(),
                    self._weight.data_ptr(),
                    out.data_ptr(),
                    self.tokens,
                    self.features,
                    _DTYPES[self.dtype],
                    self.epsilon,
                    _stream(self.device),
                )
            )
        return out
