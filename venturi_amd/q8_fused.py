"""Fused W8A8 projections: two or three Q8 matrices of one K against one A8 activation pack.

Public surface of the reference's ops/q8_fused.py (``OutputDescriptor``,
``PreparedQ8Fused.run(x, *, outputs, workspace, packed=False)``,
``prepare_q8_fused(residents, *, tokens, residual_compensation,
output_strides=None)``), with its argument checks and messages.

A plan fixes every matrix's device pointers, row count and output stride at
prepare time (``_matrices``); ``run`` checks the caller's buffers, quantizes
the activations once into the workspace (the A8 plan's layout and size) unless
``packed``, and issues one ``venturi_q8_fused_run`` launch over a descriptor
array built from the fixed entries plus this call's output pointers. Output i
is written as [tokens][strides[i]] and holds the bytes of the reference-order
A8 projection of matrix i (``venturi_q8_dp4a_run``).
"""

import ctypes as C
from dataclasses import dataclass

import torch

from .blocks import ResidentLinear
from .operands import admit, disjoint, stream_of
from .q8_dp4a import prepare_q8_dp4a

_INT32_LIMIT = 2**31


class OutputDescriptor(C.Structure):
    """One matrix of a fused launch: the C ABI's VQFOutput (32 bytes)."""

    _fields_ = [
        ("codes", C.c_void_p),
        ("scales", C.c_void_p),
        ("out", C.c_void_p),
        ("rows", C.c_int),
        ("stride", C.c_int),
    ]


@dataclass(frozen=True)
class PreparedQ8Fused:
    residents: tuple
    base: object  # the A8 plan of the first matrix: tokens, passes, workspace size
    strides: tuple
    _run: object
    _matrices: tuple = ()  # (codes pointer, scales pointer, rows, stride) per matrix

    @property
    def workspace_bytes(self):
        return self.base.workspace_bytes

    @property
    def precision_profile(self):
        return self.base.precision_profile

    def _check_buffers(self, x, outputs, workspace):
        lead = self.residents[0]
        tokens = self.base.tokens
        if not (isinstance(outputs, (list, tuple)) and len(outputs) == len(self.residents)):
            raise ValueError("one output per fused matrix required")
        admit(x, (tokens, lead.hidden_size), torch.float16, lead.device, "x")
        admit(workspace, (self.workspace_bytes,), torch.uint8, lead.device, "workspace")
        if workspace.data_ptr() % 16 != 0:
            raise ValueError("DP4A workspace requires 16-byte alignment")
        weights = sum((m.storage_tensors for m in self.residents), ())
        disjoint(workspace, (x,) + weights)
        earlier = ()
        for out, stride in zip(outputs, self.strides):
            admit(out, (tokens, stride), torch.float16, lead.device, "out")
            disjoint(out, (x, workspace) + weights + earlier)
            earlier += (out,)

    def _descriptors(self, outputs):
        table = (OutputDescriptor * len(outputs))()
        for entry, (codes, scales, rows, stride), out in zip(table, self._matrices, outputs):
            entry.codes, entry.scales, entry.out, entry.rows, entry.stride = codes, scales, out.data_ptr(), rows, stride
        return table

    def run(self, x, *, outputs, workspace, packed=False):
        """packed=True is explicit caller-owned quantization reuse, not a pointer cache."""
        if not isinstance(packed, bool):
            raise ValueError("packed must be boolean")
        self._check_buffers(x, outputs, workspace)
        table = self._descriptors(outputs)
        lead, a8 = self.residents[0], self.base
        backend = lead.backend
        with torch.cuda.device(lead.device):
            stream = stream_of(lead.device)
            if not packed:
                backend._check(backend._native.venturi_q8_dp4a_quantize(
                    x.data_ptr(), workspace.data_ptr(), a8.workspace_bytes, a8.tokens, lead.hidden_size, a8.passes,
                    stream))
            backend._check(self._run(
                workspace.data_ptr(), a8.workspace_bytes, C.cast(table, C.c_void_p), len(table), a8.tokens,
                lead.hidden_size, lead.padded_k, a8.passes, stream))
        return outputs


def _fused_strides(values, tokens, output_strides):
    strides = tuple(m.vocab_size for m in values) if output_strides is None else tuple(output_strides)

    def valid(matrix, stride):
        return (type(stride) is int and matrix.vocab_size <= stride < _INT32_LIMIT
                and (tokens - 1) * stride + matrix.vocab_size < _INT32_LIMIT)

    if len(strides) != len(values) or not all(valid(m, s) for m, s in zip(values, strides)):
        raise ValueError("invalid fused output strides")
    return strides


def prepare_q8_fused(residents, *, tokens, residual_compensation, output_strides=None):
    """Fused plan over two or three resident Q8 matrices that share K, device and backend."""
    if not (isinstance(residents, (tuple, list)) and 2 <= len(residents) <= 3):
        raise ValueError("fused projection requires two or three resident matrices")
    values = tuple(r._payload if isinstance(r, ResidentLinear) else r for r in residents)
    # Every matrix must admit its own A8 plan (shape and dtype checks); the
    # first one's plan carries the shared token count, passes and workspace.
    plans = [prepare_q8_dp4a(m, tokens=tokens, residual_compensation=residual_compensation, route="exact")
             for m in values]
    lead = values[0]
    if not all(m.device == lead.device and m.hidden_size == lead.hidden_size and m.backend is lead.backend
               for m in values):
        raise ValueError("fused matrices require the same device, backend and K")
    if sum(m.vocab_size for m in values) >= _INT32_LIMIT - 48:
        raise ValueError("fused row sum exceeds int32")
    strides = _fused_strides(values, tokens, output_strides)
    planes = [m.row_major_planes() for m in values]
    matrices = tuple((c.data_ptr(), sc.data_ptr(), m.vocab_size, s) for (c, sc), m, s in zip(planes, values, strides))
    return PreparedQ8Fused(values, plans[0], strides, lead.backend._native.venturi_q8_fused_run, matrices)
