"""Codec registry, geometry and load-time qualification (venturi.quantization)."""

from .codecs import (
    ACTIVATION_INT8_QUALIFIED,
    CODECS,
    EXECUTION_QUALIFIED,
    FUSED_LINEAR_QUALIFIED,
    GFX950,
    Codec,
    codec_for,
    dequantize_planes,
)
from .layout import ROW_FORMATS, row_geometry, row_payload_bytes
from .linear import describe_linear_contracts, validate_linear_contracts, validate_reported_plan

__all__ = [
    "ACTIVATION_INT8_QUALIFIED",
    "CODECS",
    "Codec",
    "EXECUTION_QUALIFIED",
    "FUSED_LINEAR_QUALIFIED",
    "GFX950",
    "ROW_FORMATS",
    "codec_for",
    "dequantize_planes",
    "describe_linear_contracts",
    "row_geometry",
    "row_payload_bytes",
    "validate_linear_contracts",
    "validate_reported_plan",
]
