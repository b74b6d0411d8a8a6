"""Prepared-operator contract of the HIP backend, independent of the native library.

The public names, protocols and error texts are those of the reference's
operator contract (src/venturi/ops/backend.py:16-237), so code written against
it runs unchanged: ``OperatorSupport`` / ``BackendCapabilities`` records,
``LinearPlan`` / ``LinearWeight`` / ``OperatorBackend`` protocols, the
``Backend`` base and ``create_backend``.

Here a capability set is compiled once into a frozen set of request keys
(operation, device type, dtype, weight format, weight layout), so a support
query is one set lookup. ``create_backend`` builds the gfx950 HIP backend for
"hip" (or "cuda", the device type torch gives HIP devices); there is no CPU or
torch fallback in this package.
"""

from abc import ABC, abstractmethod
from dataclasses import dataclass, field
from typing import Protocol, runtime_checkable

import torch

# Operations whose requests name a weight format; a request without one asks for dense weights.
_WEIGHTED = frozenset(("linear", "embedding"))


class UnsupportedOperationError(ValueError):
    """The selected backend has no declared implementation for a request."""


def _fail(condition, error, message):
    if condition:
        raise error(message)


def _nonempty_text(value):
    return isinstance(value, str) and bool(value)


@dataclass(frozen=True)
class OperatorSupport:
    """One declared (operation, devices, dtypes, weight format/layout) implementation."""

    operation: str
    device_types: frozenset
    dtypes: frozenset
    weight_format: str | None = None
    weight_layout: str | None = None
    materializes_weights: bool = False

    def __post_init__(self):
        devices, dtypes = frozenset(self.device_types), frozenset(self.dtypes)
        object.__setattr__(self, "device_types", devices)
        object.__setattr__(self, "dtypes", dtypes)
        _fail(not (_nonempty_text(self.operation) and devices and dtypes), ValueError,
              "Operator support requires an operation, devices and dtypes")
        _fail(not all(_nonempty_text(d) for d in devices), ValueError, "Device types must be nonempty strings")
        _fail(not all(isinstance(d, torch.dtype) for d in dtypes), TypeError,
              "Capability dtypes must be torch.dtype values")
        _fail(self.weight_format is None and self.weight_layout is not None, ValueError,
              "A weight layout requires an explicit format")
        _fail(any(v is not None and not _nonempty_text(v) for v in (self.weight_format, self.weight_layout)),
              ValueError, "Weight format/layout must be nonempty strings")
        _fail(not isinstance(self.materializes_weights, bool), TypeError, "Weight materialization flag must be bool")

    def keys(self):
        """Every request key this declaration satisfies."""
        return {(self.operation, d, t, self.weight_format, self.weight_layout)
                for d in self.device_types for t in self.dtypes}


@dataclass(frozen=True)
class BackendCapabilities:
    """Allocation-free implementation metadata: which requests a backend declares."""

    implementation: str
    operators: tuple
    reference: bool = False
    cuda_graphs: bool = False
    _keys: frozenset = field(default=frozenset(), init=False, repr=False, compare=False)

    def __post_init__(self):
        operators = tuple(self.operators)
        object.__setattr__(self, "operators", operators)
        _fail(not self.implementation or not all(isinstance(o, OperatorSupport) for o in operators), ValueError,
              "Capabilities require an implementation and typed operators")
        _fail(not (isinstance(self.reference, bool) and isinstance(self.cuda_graphs, bool)), TypeError,
              "Reference and graph capability flags must be bool")
        object.__setattr__(self, "_keys", frozenset().union(*(o.keys() for o in operators)))

    def supports(self, operation, *, dtype, device, weight_format=None, weight_layout=None):
        # torch.device only parses the name: no device is initialised here.
        if weight_format is None and operation in _WEIGHTED:
            weight_format = "dense"
        return (operation, torch.device(device).type, dtype, weight_format, weight_layout) in self._keys

    def require(self, operation, **request):
        if not self.supports(operation, **request):
            raise UnsupportedOperationError(
                f"{self.implementation} does not support {operation}: {request}; "
                "select an explicit backend/format, no automatic fallback"
            )


@runtime_checkable
class LinearPlan(Protocol):
    tokens: int
    dtype: torch.dtype
    device: torch.device
    in_features: int
    out_features: int
    workspace_bytes: int
    storage_tensors: tuple

    def run(self, x, *, out, workspace=None): ...


@runtime_checkable
class LinearWeight(Protocol):
    dtype: torch.dtype
    device: torch.device
    in_features: int
    out_features: int
    storage_tensors: tuple
    storage_nbytes: int

    def prepare(self, *, tokens) -> LinearPlan: ...

    def prepare_embedding(self, token_ids): ...


@runtime_checkable
class OperatorBackend(Protocol):
    """Structural interface: upload owns storage, prepare binds shapes, run writes outputs."""

    name: str
    capabilities: BackendCapabilities

    def resolve_device(self, device) -> torch.device: ...
    def validate_device(self, dtype, device) -> torch.device: ...
    def require(self, operation, **request): ...
    def require_linear(self, weight, *, dtype, device): ...
    def empty(self, shape, *, dtype, device) -> torch.Tensor: ...
    def synchronize(self, device): ...
    def upload_linear(self, weight, *, dtype, device) -> LinearWeight: ...
    def upload_rmsnorm(self, weight, *, dtype, device, epsilon): ...
    def prepare_linear(self, weight, *, tokens, dtype, device) -> LinearPlan: ...
    def prepare_rmsnorm(self, weight, *, tokens, dtype, device, epsilon): ...


class Backend(ABC):
    """Optional base of concrete backends: capability checks on top of abstract upload/prepare."""

    @property
    @abstractmethod
    def capabilities(self) -> BackendCapabilities: ...

    def require(self, operation, **request):
        self.capabilities.require(operation, **request)

    def require_linear(self, weight, *, dtype, device):
        request = {"dtype": dtype, "device": device, "weight_format": weight.format,
                   "weight_layout": getattr(weight, "layout", None)}
        self.require("linear", **request)

    @abstractmethod
    def resolve_device(self, device) -> torch.device: ...

    @abstractmethod
    def validate_device(self, dtype, device) -> torch.device: ...

    @abstractmethod
    def empty(self, shape, *, dtype, device) -> torch.Tensor: ...

    @abstractmethod
    def synchronize(self, device): ...

    @abstractmethod
    def upload_linear(self, weight, *, dtype, device) -> LinearWeight: ...

    @abstractmethod
    def upload_rmsnorm(self, weight, *, dtype, device, epsilon): ...

    @abstractmethod
    def prepare_linear(self, weight, *, tokens, dtype, device) -> LinearPlan: ...

    @abstractmethod
    def prepare_rmsnorm(self, weight, *, tokens, dtype, device, epsilon): ...


_NATIVE_KINDS = ("hip", "cuda")


def create_backend(kind, *, library=None, q4_backend=None) -> OperatorBackend:
    """Explicit construction: loads the native library; never builds, probes devices or falls back.

    ``library`` defaults to the in-tree build. ``q4_backend`` is accepted for
    signature compatibility: Q4 runs in the same library and needs no plugin.
    """
    if kind not in _NATIVE_KINDS:
        detail = ("The CPU torch reference backend is not part of venturi_amd; select 'hip' explicitly"
                  if kind == "torch" else f"Backend {kind!r} is not implemented; select 'hip' explicitly")
        raise UnsupportedOperationError(detail)
    from .blocks import HipBackend

    return HipBackend(library)
