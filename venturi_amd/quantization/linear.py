"""Load-time numerical and capability checks of row QuantLinear.

Public functions and error texts of the reference's quantization/linear.py
(lines 16-122): ``validate_linear_contracts(spec, weights)``,
``describe_linear_contracts(weights, profile, implementation)`` and
``validate_reported_plan(fmt, profile, architecture, values)``. The gfx950
capability (torch reports (9, 5)) is admitted beside the reference's (7, 0)
and (8, 9). Unsupported combinations raise; nothing falls back.

The spec is read once into a ``_Policy`` record; each check is a rule that
yields the first message it finds (``_binding_rules`` per quantized matrix,
then ``_model_rules`` for the whole plan), and the first message raises.
"""

from dataclasses import dataclass

import torch

from .codecs import (
    ACTIVATION_INT8_QUALIFIED,
    EXECUTION_QUALIFIED,
    FUSED_LINEAR_QUALIFIED,
    GFX950,
    codec_for,
)

SUPPORTED_ARCHITECTURES = ((7, 0), (8, 9), GFX950)

# Family numbers of the native plan-info tuple [bits, group, passes, family, min_hmma_tokens, shadow].
_FAMILY_NAMES = ("direct", "chunked-dense", "activation-int8")
_PASSES = {"fp16": 0, "int8": 1}


@dataclass(frozen=True)
class _Policy:
    arch: tuple
    profile: str
    implementation: str
    resident_fp16_single_device: bool
    dequant_resident: bool


def _policy(spec):
    plain = (spec.dtype == torch.float16 and spec.weight_mode == "resident"
             and spec.tensor_parallel_device is None and spec.stage_range is None)
    return _Policy(tuple(torch.cuda.get_device_capability(spec.target)), spec.projection_profile,
                   spec.linear_implementation, plain, spec.dequant_resident)


def _int8_kernel_exists(bits, arch):
    # Q8 everywhere; the SM70 build also has a Q5 int8 kernel.
    return bits == 8 or (bits == 5 and arch == (7, 0))


def _binding_rules(policy, fmt, codec):
    """Messages for one quantized matrix, in the order they are decided."""
    arch = policy.arch
    if fmt not in EXECUTION_QUALIFIED.get(arch, ()):
        yield "Matrix codec is not execution-qualified on this architecture: " + fmt
    if policy.profile == "int8" and fmt not in ACTIVATION_INT8_QUALIFIED.get(arch, ()):
        yield "One-pass int8 model execution qualification pending: " + fmt
    if policy.implementation == "fused" and fmt not in FUSED_LINEAR_QUALIFIED.get(arch, ()):
        yield "Fused model execution qualification pending: " + fmt
    if codec.bits != 8:
        if not policy.resident_fp16_single_device:
            yield "row-codec matrices require resident single-device FP16 without TP/PP"
        if policy.profile not in ("fp16", "int8"):
            yield "Residual activation policy requires Q8 matrices"
    if policy.profile == "int8" and not _int8_kernel_exists(codec.bits, arch):
        yield "Explicit int8 activation policy has no qualified kernel for " + fmt


def _model_rules(policy, row_codec_count, any_q8):
    if policy.implementation == "dequant":
        if row_codec_count == 0:
            yield "dequant reference requires Q4/Q5/Q6 matrices"
        if not policy.resident_fp16_single_device:
            yield "dequant reference requires resident single-device FP16 without TP/PP"
    if policy.dequant_resident and any_q8:
        yield "FP16 shadow requires only Q4/Q5/Q6 matrices"


def _raise_first(messages):
    for message in messages:
        raise ValueError(message)


def validate_linear_contracts(spec, weights):
    policy = _policy(spec)
    if policy.arch not in SUPPORTED_ARCHITECTURES:
        raise ValueError("Unsupported QuantLinear architecture")
    bits_seen = []
    for binding in weights.plan.bindings:
        codec = codec_for(binding.format)
        if codec.quantized:
            _raise_first(_binding_rules(policy, binding.format, codec))
            bits_seen.append(codec.bits)
    _raise_first(_model_rules(policy, sum(b != 8 for b in bits_seen), 8 in bits_seen))


def _weight_decode(bits, profile, implementation):
    # W4/5/6A16 rounds every weight to fp16(q * scale), except the Q4 fused research GEMV.
    rounded = bits in (4, 5, 6) and profile == "fp16" and not (bits == 4 and implementation == "fused")
    return "fp16-rounded-q-times-scale" if rounded else "fp32-scaled-integer-products"


def describe_linear_contracts(weights, profile, implementation="auto"):
    """Per-format numerical description of a model's quantized matrices; no device access."""
    formats = sorted({b.format for b in weights.plan.bindings if codec_for(b.format).quantized})
    return {fmt: {"layout": codec_for(fmt).layout,
                  "activation_policy": profile,
                  "weight_decode": _weight_decode(codec_for(fmt).bits, profile, implementation),
                  "accumulation": "fp32; implementation-dependent association"}
            for fmt in formats}


def validate_reported_plan(fmt, profile, architecture, values):
    """Checks the native plan-info tuple against the codec and policy, and names the family it selected."""
    codec = codec_for(fmt)
    passes = _PASSES.get(profile, 2)
    if len(values) != 6 or tuple(values[:3]) != (codec.bits, codec.group, passes):
        raise RuntimeError("Native QuantLinear numerical/codec contract mismatch")
    family = int(values[3])
    if family not in (0, 1, 2):
        raise RuntimeError("Native QuantLinear family/activation-policy mismatch")
    if family == 0 and fmt not in FUSED_LINEAR_QUALIFIED.get(tuple(architecture), ()):
        raise ValueError("Native backend selected an unqualified direct/fused family: " + fmt)
    if family == 1 and (codec.bits not in (4, 5, 6) or passes != 0):
        raise RuntimeError("Native dense row-codec plan contract mismatch")
    if family == 2 and passes == 0:
        raise RuntimeError("Native QuantLinear family/activation-policy mismatch")
    return "resident-fp16-shadow" if values[5] else _FAMILY_NAMES[family]
