"""HIP backend: uploads, shape plans and explicit-buffer execution on gfx950.

Mirrors the reference's prepared-operator layer (venturi.ops.blocks,
blocks.py:27-581): ``ResidentLinear`` / ``ResidentRMSNorm`` records, the same
operand guards (exact shape, dtype and device, contiguity, no aliasing,
inference only), and plans whose ``run`` performs no allocation,
synchronisation or implicit cast, so they can be captured in HIP graphs.
Every kernel is called through the C ABI of libventuri_ops.so.
"""

from dataclasses import dataclass

import torch

from . import native
from .backend import Backend, BackendCapabilities, OperatorSupport, UnsupportedOperationError
from .operands import DTYPE_CODES, admit, disjoint, epsilon as admit_epsilon, extents, stream_of
from .weights import DenseWeight, Q4RowSplitWeight, Q8RowSplitWeight

Q8_ROUTES = ("auto", "exact", "mfma", "dense")


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
        extents(tokens, self.in_features)
        self._backend.validate_device(self.dtype, self.device)
        return self._backend.bind_linear(self, tokens=tokens, route=route)

    def prepare_swiglu(self, *, tokens):
        """Fused gate+up projection and SwiGLU for a Q8 [2 * inter, hidden] weight, gate rows
        first (an extension: the native runtime runs the projection, then SwiGLU). The plan's
        output is [tokens, inter]."""
        from .vocabulary import ResidentQ8Vocabulary

        extents(tokens, self.in_features)
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
        extents(tokens, self.features)
        self._backend.validate_device(self.dtype, self.device)
        return self._backend.bind_rmsnorm(self, tokens=tokens)


def _capabilities():
    devices = frozenset(("cuda",))
    quant = frozenset((torch.float16, torch.bfloat16))
    floating = frozenset((torch.float16, torch.bfloat16, torch.float32))
    operators = [
        OperatorSupport("rmsnorm", devices, floating),
        OperatorSupport("swiglu", devices, floating),
        OperatorSupport("add", devices, floating),
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
        if dtype not in DTYPE_CODES:
            raise ValueError("Native blocks require FP16, BF16 or FP32")
        return self.resolve_device(device)

    def resolve_device(self, device):
        """The concrete gfx950 device a request names; refused during graph capture."""
        requested = torch.device(device)
        if requested.type != "cuda":
            raise ValueError("HipBackend requires an explicit GPU device")
        with torch.cuda.device(requested):
            index = torch.cuda.current_device()
            capturing = torch.cuda.is_current_stream_capturing()
        if capturing:
            raise RuntimeError("Preparation must run outside graph capture")
        target = torch.device("cuda", index)
        if not is_gfx950(target):
            raise ValueError("libventuri_ops.so is built for gfx950 (MI355X) only")
        return target

    def empty(self, shape, *, dtype, device):
        """Uninitialised device tensor for caller-owned buffers (outputs, workspaces)."""
        valid_shape = isinstance(shape, (list, tuple)) and all(type(d) is int and 0 <= d < 2**31 for d in shape)
        if not valid_shape:
            raise ValueError("Allocation shape must contain nonnegative int32 extents")
        if not isinstance(dtype, torch.dtype):
            raise TypeError("Allocation requires an explicit torch.dtype")
        # Floating buffers must be a dtype the kernels take; byte and index buffers only a device.
        check = self.validate_device if dtype.is_floating_point else lambda _, d: self.resolve_device(d)
        return torch.empty(tuple(shape), dtype=dtype, device=check(dtype, device))

    def _launch(self, entry, device, *operands):
        """Calls one C entry point on `device`'s current stream: tensors pass as data pointers,
        every other operand as it is; a -1 return raises the library's message."""
        arguments = [v.data_ptr() if isinstance(v, torch.Tensor) else v for v in operands]
        with torch.cuda.device(device):
            self._check(getattr(self._native, entry)(*arguments, stream_of(device)))

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
        extents(n, k)
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
                    source.data_ptr(), codes.data_ptr(), scales.data_ptr(), n, k, padded, DTYPE_CODES[source.dtype],
                    stream_of(target),
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
        extents(n, k)
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
                    source.data_ptr(), codes.data_ptr(), scales.data_ptr(), n, k, padded, DTYPE_CODES[source.dtype],
                    stream_of(target),
                )
            )
        return Q4RowSplitWeight(codes, scales, k)

    def bind_linear(self, resident, *, tokens, route="auto"):
        extents(tokens, 1)
        if resident._backend is not self:
            raise ValueError("Resident weight belongs to a different backend instance")
        from .vocabulary import ResidentQ8Vocabulary

        if isinstance(resident._payload, ResidentQ8Vocabulary):
            return _Q8Linear(resident._payload.prepare(tokens=tokens, route=route))
        return resident._payload.prepare(tokens=tokens, route=route)

    def prepare_linear(self, weight, *, tokens, dtype, device):
        extents(tokens, 1)
        return self.upload_linear(weight, dtype=dtype, device=device).prepare(tokens=tokens)

    # -- rmsnorm and the elementwise blocks of the gated MLP ---------------
    def upload_rmsnorm(self, weight, *, dtype, device, epsilon):
        """Owned fp32 copy of a norm vector (the kernel reads gamma in fp32 for every dtype)."""
        is_vector = isinstance(weight, torch.Tensor) and weight.ndim == 1 and weight.is_floating_point()
        if not is_vector:
            raise ValueError("RMSNorm weight must be a floating-point vector")
        extents(1, weight.numel())
        eps = admit_epsilon(epsilon)
        target = self.validate_device(dtype, device)
        with torch.cuda.device(target):
            gamma = torch.empty(weight.numel(), dtype=torch.float32, device=target)
            gamma.copy_(weight.detach())
            finite = bool(torch.isfinite(gamma).all())  # synchronises: the copy is complete
        if not finite:
            raise ValueError("RMSNorm weight must be finite in FP32")
        return ResidentRMSNorm(self, gamma, dtype, eps)

    def _owned_by_me(self, resident):
        if resident._backend is not self:
            raise ValueError("Resident weight belongs to a different backend instance")

    def bind_rmsnorm(self, resident, *, tokens):
        extents(tokens, 1)
        self._owned_by_me(resident)
        return _RMSNorm(self, resident._weight, tokens, resident.dtype, resident.epsilon)

    def prepare_rmsnorm(self, weight, *, tokens, dtype, device, epsilon):
        extents(tokens, 1)
        return self.upload_rmsnorm(weight, dtype=dtype, device=device, epsilon=epsilon).prepare(tokens=tokens)

    def prepare_swiglu(self, *, tokens, features, dtype, device):
        """Plan of out = cast((a * sigmoid(a)) * b) over [tokens, features] (blocks.py:565-572)."""
        shape = extents(tokens, features)
        return _Pointwise(self, shape, dtype, self.validate_device(dtype, device), "venturi_swiglu_run")

    def prepare_add(self, *, tokens, features, dtype, device):
        """Plan of out = cast(a + b) over [tokens, features] (blocks.py:574-581)."""
        shape = extents(tokens, features)
        return _Pointwise(self, shape, dtype, self.validate_device(dtype, device), "venturi_add_run")


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
    """RMSNorm plan (blocks.py:789-823): statistics in the reference's reduction order."""

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
        for name, tensor in (("x", x), ("out", out)):
            admit(tensor, shape, self.dtype, self.device, name)
        disjoint(out, (x, self._weight))
        self._backend._launch("venturi_rms_run", self.device, x, self._weight, out, self.tokens, self.features,
                              DTYPE_CODES[self.dtype], self.epsilon)
        return out


@dataclass(frozen=True)
class _Pointwise:
    """Elementwise plan over three [tokens, features] tensors of one dtype (blocks.py:848-876).

    ``out`` may be ``a`` or ``b`` itself (the gated MLP writes SwiGLU over its
    gate buffer), never a partial overlap.
    """

    _backend: HipBackend
    shape: tuple
    dtype: torch.dtype
    device: torch.device
    entry: str
    workspace_bytes = 0

    @property
    def swiglu(self):
        return self.entry == "venturi_swiglu_run"

    def run(self, a, b, *, out):
        for name, tensor in (("a", a), ("b", b), ("out", out)):
            admit(tensor, self.shape, self.dtype, self.device, name)
        disjoint(out, (a, b), allow_inplace=True)
        self._backend._launch(self.entry, self.device, a, b, out, a.numel(), DTYPE_CODES[self.dtype])
        return out
