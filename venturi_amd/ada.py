"""The Q4 linear plugin interface (reference ops/ada.py:20-204) over libventuri_ops.so.

``AdaBackend`` keeps the reference plugin's objects and checks:
``upload_linear`` copies the planes once, ``ResidentQ4Weight.prepare`` asks
``venturi_q4_prepare`` for the native route (auto/generic -> 0) and
``PreparedLinear.run`` calls ``venturi_q4_run``, the FP32-weight SIMT order of
q4_linear.cu:21-56 (bit-identical here). Errors carry the plugin's own
thread-local message (``venturi_ada_error``). Device qualification is gfx950
instead of compute capability 8.9.
"""

from dataclasses import dataclass
from pathlib import Path

import torch

from . import native
from .blocks import _overlaps, is_gfx950
from .weights import Q4RowSplitWeight


class AdaBackend:
    """Q4 plugin; loading neither compiles code nor allocates GPU memory."""

    name = "venturi-ada"
    abi_version = 2

    def __init__(self, library=None):
        self._native = native.load(library)
        self.library = Path(self._native.path)
        if self._native.venturi_ada_abi() != self.abi_version:
            raise RuntimeError("Venturi Ada native ABI mismatch; rebuild the backend")

    def _error(self):
        return RuntimeError(self._native.venturi_ada_error().decode("utf-8", "replace"))

    def upload_linear(self, weight, *, device="cuda:0"):
        """Copy Q4 planes once; resident storage can bind multiple shapes/dtypes."""
        if not isinstance(weight, Q4RowSplitWeight):
            raise TypeError("Venturi Ada currently supports Q4RowSplitWeight only")
        weight.validate()
        target = self._device(device)
        with torch.cuda.device(target):
            codes = weight.codes.detach().to(target, copy=True)
            scales = weight.scales.detach().to(target, copy=True)
            if not bool(torch.isfinite(scales).all()):
                raise ValueError("scales must be finite")
            owned = Q4RowSplitWeight(codes, scales, weight.in_features)
            torch.cuda.current_stream(target).synchronize()
        return ResidentQ4Weight(self, owned)

    def _device(self, device):
        target = torch.device(device)
        if target.type != "cuda":
            raise ValueError("Ada execution requires an explicit GPU device")
        with torch.cuda.device(target):
            target = torch.device("cuda", torch.cuda.current_device())
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("prepare_linear must run outside graph capture")
            if not is_gfx950(target):
                raise ValueError("This Q4 plugin build requires gfx950")
        return target


def _configuration(tokens, dtype, route):
    if type(tokens) is not int or not 0 < tokens <= 4 * 65535:
        raise ValueError("tokens must be an integer in [1, 262140]")
    if dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("activations and output must be float16 or bfloat16")
    if route not in ("auto", "generic"):
        raise ValueError("route must be auto or generic; tuned/mma were removed")


@dataclass(frozen=True)
class ResidentQ4Weight:
    """Owned read-only-by-contract Q4 planes; plans retain them."""

    _backend: AdaBackend
    _weight: Q4RowSplitWeight

    @property
    def storage_tensors(self):
        return (self._weight.codes, self._weight.scales)

    @property
    def storage_nbytes(self):
        return sum(t.numel() * t.element_size() for t in self.storage_tensors)

    def prepare(self, *, tokens, dtype=torch.bfloat16, route="auto"):
        _configuration(tokens, dtype, route)
        target = self._backend._device(self._weight.codes.device)
        with torch.cuda.device(target):
            native_route = self._backend._native.venturi_q4_prepare(
                self._weight.out_features,
                self._weight.in_features,
                tokens,
                int(dtype == torch.bfloat16),
                {"auto": -1, "generic": 0}[route],
            )
            if native_route < 0:
                raise self._backend._error()
        return PreparedLinear(self._backend, self._weight, tokens, dtype, native_route)


@dataclass(frozen=True)
class PreparedLinear:
    """Fixed-shape Linear out[T, N] = x[T, K] @ W[N, K]^T, caller-owned output."""

    workspace_bytes = 0

    _backend: AdaBackend
    _weight: Q4RowSplitWeight
    tokens: int
    dtype: torch.dtype
    _native_route: int

    @property
    def device(self):
        return self._weight.codes.device

    @property
    def in_features(self):
        return self._weight.in_features

    @property
    def out_features(self):
        return self._weight.out_features

    @property
    def route(self):
        if self._native_route != 0:
            raise RuntimeError("Unexpected native Q4 implementation")
        return "generic-simt"

    def empty_output(self):
        """Explicit allocation helper; call before timing or graph capture."""
        return torch.empty((self.tokens, self.out_features), dtype=self.dtype, device=self.device)

    def run(self, x, *, out):
        if torch.is_grad_enabled() and (x.requires_grad or out.requires_grad):
            raise ValueError("Venturi Ada is inference-only; disable gradients")
        self._weight.validate()
        for name, tensor, shape in (
            ("x", x, (self.tokens, self.in_features)),
            ("out", out, (self.tokens, self.out_features)),
        ):
            if tensor.shape != shape or tensor.dtype != self.dtype or tensor.device != self.device:
                raise ValueError(f"{name} must have shape {shape}, dtype {self.dtype}, device {self.device}")
            if not tensor.is_contiguous():
                raise ValueError(f"{name} must be contiguous; no implicit copy is performed")
            if tensor.data_ptr() % 2:
                raise ValueError(f"{name} requires 2-byte alignment")
        for operand in (x, self._weight.codes, self._weight.scales):
            if _overlaps(out, operand):
                raise ValueError("output must not alias input or weight storage")
        with torch.cuda.device(self.device):
            stream = torch.cuda.current_stream(self.device)
            result = self._backend._native.venturi_q4_run(
                x.data_ptr(),
                self._weight.codes.data_ptr(),
                self._weight.scales.data_ptr(),
                out.data_ptr(),
                self.out_features,
                self.in_features,
                self._weight.padded_k,
                self.tokens,
                int(self.dtype == torch.bfloat16),
                self._native_route,
                stream.cuda_stream,
            )
            if result < 0:
                raise self._backend._error()
        return out
