"""Prepared-operator contract, independent of any native library.

Mirrors venturi.ops.backend (reference backend.py:16-237): the same
``OperatorSupport``/``BackendCapabilities`` records and the ``LinearPlan`` /
``LinearWeight`` / ``OperatorBackend`` protocols. ``create_backend`` builds
this package's HIP backend for kind "hip" (or "cuda", the device type torch
uses for HIP devices). There is no implicit CPU fallback: the reference's
Torch reference backend is not part of this package.
"""

from abc import ABC, abstractmethod
from dataclasses import dataclass
from typing import Protocol, runtime_checkable

import torch


class UnsupportedOperationError(ValueError):
    """The selected backend has no declared implementation for a request."""


@dataclass(frozen=True)
class OperatorSupport:
    operation: str
    device_types: frozenset
    dtypes: frozenset
    weight_format: str | None = None
    weight_layout: str | None = None
    materializes_weights: bool = False

    def __post_init__(self):
        object.__setattr__(self, "device_types", frozenset(self.device_types))
        object.__setattr__(self, "dtypes", frozenset(self.dtypes))
        if not isinstance(self.operation, str) or not self.operation or not self.device_types or not self.dtypes:
            raise ValueError("Operator support requires an operation, devices and dtypes")
        if any(not isinstance(d, str) or not d for d in self.device_types):
            raise ValueError("Device types must be nonempty strings")
        if any(not isinstance(d, torch.dtype) for d in self.dtypes):
            raise TypeError("Capability dtypes must be torch.dtype values")
        if self.weight_layout is not None and self.weight_format is None:
            raise ValueError("A weight layout requires an explicit format")
        for value in (self.weight_format, self.weight_layout):
            if value is not None and (not isinstance(value, str) or not value):
                raise ValueError("Weight format/layout must be nonempty strings")
        if type(self.materializes_weights) is not bool:
            raise TypeError("Weight materialization flag must be bool")


@dataclass(frozen=True)
class BackendCapabilities:
    implementation: str
    operators: tuple
    reference: bool = False
    cuda_graphs: bool = False

    def __post_init__(self):
        object.__setattr__(self, "operators", tuple(self.operators))
        if not self.implementation or any(not isinstance(o, OperatorSupport) for o in self.operators):
            raise ValueError("Capabilities require an implementation and typed operators")
        if type(self.reference) is not bool or type(self.cuda_graphs) is not bool:
            raise TypeError("Reference and graph capability flags must be bool")

    def supports(self, operation, *, dtype, device, weight_format=None, weight_layout=None):
        kind = torch.device(device).type  # metadata only; no device initialisation
        if operation in ("linear", "embedding") and weight_format is None:
            weight_format = "dense"
        return any(
            o.operation == operation
            and kind in o.device_types
            and dtype in o.dtypes
            and weight_format == o.weight_format
            and weight_layout == o.weight_layout
            for o in self.operators
        )

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
    """Optional base class for the public contract (backend.py:153-214)."""

    @property
    @abstractmethod
    def capabilities(self) -> BackendCapabilities: ...

    def require(self, operation, **request):
        self.capabilities.require(operation, **request)

    def require_linear(self, weight, *, dtype, device):
        self.require(
            "linear",
            dtype=dtype,
            device=device,
            weight_format=weight.format,
            weight_layout=getattr(weight, "layout", None),
        )

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


def create_backend(kind, *, library=None, q4_backend=None) -> OperatorBackend:
    """Explicit construction only: loads the native library, never builds or probes devices.

    ``library`` defaults to the in-tree build. ``q4_backend`` is accepted for
    signature compatibility; Q4 is native to this backend and needs no plugin.
    """
    if kind in ("hip", "cuda"):
        from .blocks import HipBackend

        return HipBackend(library)
    if kind == "torch":
        raise UnsupportedOperationError(
            "The CPU torch reference backend is not part of venturi_amd; select 'hip' explicitly"
        )
    raise UnsupportedOperationError(f"Backend {kind!r} is not implemented; select 'hip' explicitly")
