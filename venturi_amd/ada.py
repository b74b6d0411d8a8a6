"""The Q4 linear plugin interface (the reference's ops/ada.py) over libventuri_ops.so.

Public objects and texts of the reference plugin: ``AdaBackend`` (ABI 2,
``upload_linear``), ``ResidentQ4Weight.prepare(tokens=, dtype=, route=)`` and
``PreparedLinear.run(x, out=)``. The plugin's entry points live in the same
library as the blocks ABI: ``venturi_q4_prepare`` admits a native route (auto
and generic map to route 0, the FP32-weight SIMT order of
q4_linear.cu:21-56, bit-identical here) and ``venturi_q4_run`` executes it;
failures carry the plugin's own thread-local message (``venturi_ada_error``).
Device qualification is gfx950 instead of compute capability 8.9.

A prepared plan keeps its launch arguments (weight pointers, geometry, dtype
and route codes) as one tuple built at prepare time; ``run`` checks the two
caller buffers against the plan and inserts their pointers.
"""

from dataclasses import dataclass
from pathlib import Path

import torch

from . import native
from .blocks import is_gfx950
from .operands import overlapping
from .weights import Q4RowSplitWeight

_MAX_TOKENS = 4 * 65535
_ROUTE_CODES = {"auto": -1, "generic": 0}
_DTYPE_CODES = {torch.float16: 0, torch.bfloat16: 1}


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

    def _device(self, device):
        """The concrete gfx950 device for `device`, outside graph capture."""
        target = torch.device(device)
        if target.type != "cuda":
            raise ValueError("Ada execution requires an explicit GPU device")
        with torch.cuda.device(target):
            index = torch.cuda.current_device()
            capturing = torch.cuda.is_current_stream_capturing()
        if capturing:
            raise RuntimeError("prepare_linear must run outside graph capture")
        target = torch.device("cuda", index)
        if not is_gfx950(target):
            raise ValueError("This Q4 plugin build requires gfx950")
        return target

    def upload_linear(self, weight, *, device="cuda:0"):
        """Copies the Q4 planes once; the resident storage serves plans of any shape and dtype."""
        if not isinstance(weight, Q4RowSplitWeight):
            raise TypeError("Venturi Ada currently supports Q4RowSplitWeight only")
        weight.validate()
        target = self._device(device)
        with torch.cuda.device(target):
            planes = [t.detach().to(target, copy=True) for t in (weight.codes, weight.scales)]
            if not bool(torch.isfinite(planes[1]).all()):
                raise ValueError("scales must be finite")
            torch.cuda.current_stream(target).synchronize()
        return ResidentQ4Weight(self, Q4RowSplitWeight(*planes, weight.in_features))


def _admit(tokens, dtype, route):
    if type(tokens) is not int or not 0 < tokens <= _MAX_TOKENS:
        raise ValueError("tokens must be an integer in [1, 262140]")
    if dtype not in _DTYPE_CODES:
        raise ValueError("activations and output must be float16 or bfloat16")
    if route not in _ROUTE_CODES:
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
        _admit(tokens, dtype, route)
        w, lib = self._weight, self._backend._native
        target = self._backend._device(w.codes.device)
        with torch.cuda.device(target):
            chosen = lib.venturi_q4_prepare(w.out_features, w.in_features, tokens, _DTYPE_CODES[dtype],
                                            _ROUTE_CODES[route])
        if chosen < 0:
            raise self._backend._error()
        launch = (w.codes.data_ptr(), w.scales.data_ptr(), w.out_features, w.in_features, w.padded_k, tokens,
                  _DTYPE_CODES[dtype], chosen)
        return PreparedLinear(self._backend, w, tokens, dtype, chosen, launch)


@dataclass(frozen=True)
class PreparedLinear:
    """Fixed-shape out[T, N] = x[T, K] @ W[N, K]^T without bias; caller-owned output."""

    workspace_bytes = 0

    _backend: AdaBackend
    _weight: Q4RowSplitWeight
    tokens: int
    dtype: torch.dtype
    _native_route: int
    _launch: tuple = ()  # (codes, scales, n, k, padded, tokens, dtype code, route) for venturi_q4_run

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

    def _check(self, name, tensor, features):
        shape = (self.tokens, features)
        if tensor.shape != shape or tensor.dtype != self.dtype or tensor.device != self.device:
            raise ValueError(f"{name} must have shape {shape}, dtype {self.dtype}, device {self.device}")
        if not tensor.is_contiguous():
            raise ValueError(f"{name} must be contiguous; no implicit copy is performed")
        if tensor.data_ptr() % 2:
            raise ValueError(f"{name} requires 2-byte alignment")

    def run(self, x, *, out):
        if torch.is_grad_enabled() and (x.requires_grad or out.requires_grad):
            raise ValueError("Venturi Ada is inference-only; disable gradients")
        self._weight.validate()
        self._check("x", x, self.in_features)
        self._check("out", out, self.out_features)
        if any(overlapping(out, t) for t in (x, self._weight.codes, self._weight.scales)):
            raise ValueError("output must not alias input or weight storage")
        codes, scales, n, k, padded, tokens, dtype_code, route = self._launch
        with torch.cuda.device(self.device):
            status = self._backend._native.venturi_q4_run(
                x.data_ptr(), codes, scales, out.data_ptr(), n, k, padded, tokens, dtype_code, route,
                torch.cuda.current_stream(self.device).cuda_stream)
        if status < 0:
            raise self._backend._error()
        return out
