"""RMSNorm fused with per-32-group int8 activation quantization.

The reference exposes this producer only to its native runtime
(venturi_rms_q8_quantize, q8_rms_producer.cuh:67-84, two passes). This plan
wraps the same C entry and its one-or-two-pass extension: it writes the A8
workspace consumed by ``PreparedQ8DP4A.project`` and, optionally, the fp16
normalised activations.
"""

from dataclasses import dataclass

import torch

from .blocks import ResidentRMSNorm
from .operands import admit, disjoint, extents, stream_of


@dataclass(frozen=True)
class PreparedRMSQ8:
    norm: ResidentRMSNorm
    tokens: int
    passes: int
    workspace_bytes: int

    def run(self, x, *, workspace, intermediate=None):
        n = self.norm
        k = n.features
        admit(x, (self.tokens, k), torch.float16, n.device, "x")
        admit(workspace, (self.workspace_bytes,), torch.uint8, n.device, "workspace")
        disjoint(workspace, (x, n._weight))
        if intermediate is not None:
            admit(intermediate, (self.tokens, k), torch.float16, n.device, "intermediate")
            disjoint(intermediate, (x, n._weight, workspace))
        if workspace.data_ptr() % 16:
            raise ValueError("A8 workspace requires 16-byte alignment")
        lib = n._backend._native
        with torch.cuda.device(n.device):
            n._backend._check(
                lib.venturi_rms_q8_quantize_passes(
                    x.data_ptr(), n._weight.data_ptr(), workspace.data_ptr(), self.workspace_bytes, self.tokens, k,
                    n.epsilon, self.passes, intermediate.data_ptr() if intermediate is not None else None,
                    stream_of(n.device),
                )
            )
        return workspace


def prepare_rms_q8(norm, *, tokens, residual_compensation):
    """Plan RMSNorm -> fp16 -> A8 for ``tokens`` rows of an fp16 ResidentRMSNorm."""
    if not isinstance(norm, ResidentRMSNorm):
        raise ValueError("RMS/A8 requires a resident RMSNorm")
    if type(residual_compensation) is not bool:
        raise ValueError("Explicit boolean residual_compensation required")
    if norm.dtype != torch.float16:
        raise ValueError("RMS/A8 requires FP16 activations")
    extents(tokens, norm.features)
    norm._backend.validate_device(norm.dtype, norm.device)
    passes = 2 if residual_compensation else 1
    size = norm._backend._native.venturi_q8_dp4a_bytes(tokens, norm.features, passes)
    if not size:
        norm._backend._check(-1)
    return PreparedRMSQ8(norm, tokens, passes, size)
