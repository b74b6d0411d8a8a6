"""MI355X (gfx950) quantized-linear path: Q8/Q4 row codecs, A8 and W4A16 kernels.

A drop-in for the reference's QuantLinear operator layer (venturi.ops) on the
quantized-linear path: the same descriptors, backend protocol and plan API,
executed by hand-written HIP kernels in libventuri_ops.so.
"""

from .backend import (
    Backend,
    BackendCapabilities,
    LinearPlan,
    LinearWeight,
    OperatorBackend,
    OperatorSupport,
    UnsupportedOperationError,
    create_backend,
)
from .weights import DenseWeight, Q4RowSplitWeight, Q8RowSplitWeight

__all__ = [
    "Backend",
    "BackendCapabilities",
    "DenseWeight",
    "HipBackend",
    "LinearPlan",
    "LinearWeight",
    "OperatorBackend",
    "OperatorSupport",
    "Q4RowSplitWeight",
    "Q8RowSplitWeight",
    "UnsupportedOperationError",
    "create_backend",
    "prepare_q8_dp4a",
    "prepare_q8_fused",
    "prepare_rms_q8",
    "quantize_q4_rtn",
    "decode_q4_fp16",
]


def __getattr__(name):
    # Deferred so that importing the descriptors never loads the native library.
    if name == "HipBackend":
        from .blocks import HipBackend

        return HipBackend
    if name == "prepare_q8_dp4a":
        from .q8_dp4a import prepare_q8_dp4a

        return prepare_q8_dp4a
    if name == "prepare_q8_fused":
        from .q8_fused import prepare_q8_fused

        return prepare_q8_fused
    if name == "prepare_rms_q8":
        from .rms_quant import prepare_rms_q8

        return prepare_rms_q8
    if name in ("quantize_q4_rtn", "decode_q4_fp16"):
        from . import q4

        return getattr(q4, name)
    raise AttributeError(name)
