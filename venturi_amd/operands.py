"""Operand admission for prepared plans.

Every ``run`` of a plan in this package checks its caller-owned tensors before
the launch and never copies, casts or allocates to make them fit. The rules
and their error types and texts are the reference's prepared-operator contract
(/root/reference/src/venturi/ops/blocks.py:27-68, ada.py:_overlaps), so code
written against the reference sees the same failures:

* extents (tokens, features, rows) are plain ints in [1, 2^31);
* an operand is a tensor of exactly the planned shape, dtype and device,
  contiguous, and not part of an autograd graph;
* an output or workspace shares no byte with an operand, except an output that
  is the very same tensor as an operand where the kernel allows in-place use;
* an RMSNorm epsilon is a finite, normal, positive fp32 value.
"""

import math

import torch

DTYPE_CODES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}

_INT32_END = 2**31
_F32 = torch.finfo(torch.float32)


def extents(*values):
    """The values as a tuple, each a plain int in [1, 2^31) (bools are not ints here)."""
    if not all(type(v) is int and 0 < v < _INT32_END for v in values):
        raise ValueError("tokens and features must be positive int32 values")
    return tuple(values)


def admit(tensor, shape, dtype, device, name):
    """Checks one operand against the plan's fixed (shape, dtype, device)."""
    if not isinstance(tensor, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if (tuple(tensor.shape), tensor.dtype, tensor.device) != (tuple(shape), dtype, device):
        raise ValueError(f"{name} requires shape {shape}, dtype {dtype}, device {device}")
    if not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous; no implicit copy")
    if tensor.requires_grad and torch.is_grad_enabled():
        raise ValueError("Prepared operators are inference-only")


def byte_span(tensor):
    """[first, end) byte addresses of a contiguous tensor's storage window."""
    first = tensor.data_ptr()
    return first, first + tensor.numel() * tensor.element_size()


def overlapping(a, b):
    """True when two contiguous tensors on one device share at least one byte."""
    if a.device != b.device:
        return False
    (a0, a1), (b0, b1) = byte_span(a), byte_span(b)
    return a0 < b1 and b0 < a1


def _same_view(a, b):
    return a.data_ptr() == b.data_ptr() and a.shape == b.shape and a.dtype == b.dtype


def disjoint(out, operands, *, allow_inplace=False):
    """Rejects an output / workspace that aliases any operand's bytes."""
    for operand in operands:
        if overlapping(out, operand) and not (allow_inplace and _same_view(out, operand)):
            raise ValueError("output/workspace must not alias operand storage")


def epsilon(value):
    """RMSNorm epsilon as a float: finite and within [smallest normal, largest] fp32."""
    if type(value) in (int, float) and math.isfinite(value) and _F32.tiny <= value <= _F32.max:
        return float(value)
    raise ValueError("epsilon must be finite, positive, and a normal FP32 value")


def stream_of(device):
    """The raw hipStream_t of the device's current torch stream."""
    return torch.cuda.current_stream(device).cuda_stream
