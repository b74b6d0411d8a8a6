"""The native runtime's QuantLinear plan table over the C ABI.

``prepare_row_codec`` admits a kernel family once from (bits, group,
precision, dtype, implementation), as rowcodec::prepare does in the reference
(row_codec_dispatch.cuh:6-64), and ``RowCodecPlan.project`` runs one matrix
the way Model::project does (qwen_runtime.cuh:348-390): Q8 A16 directly, A8
through the activation pack in a caller-owned workspace, Q4/Q5/Q6 A16 through
the W*A16 contract GEMM.
"""

import ctypes as C
from dataclasses import dataclass

from . import native

PRECISIONS = {"w16a16": 0, "wxa16": 0, "wxa8": 1, "wxa8-residual": 2}
IMPLEMENTATIONS = {"auto": 0, "dequant": 1, "fused-research": 2}
PATHS = ("direct", "chunked-dense", "quantized")


class VRCPlan(C.Structure):
    _fields_ = [(name, C.c_int) for name in ("bits", "group", "precision", "dtype", "implementation", "path", "passes")]


@dataclass(frozen=True)
class RowCodecPlan:
    lib: object
    raw: VRCPlan

    @property
    def path(self):
        return PATHS[self.raw.path]

    @property
    def passes(self):
        return self.raw.passes

    def workspace_bytes(self, *, tokens, k):
        size = self.lib.venturi_rowcodec_workspace_bytes(C.byref(self.raw), tokens, k)
        if size == 0 and self.raw.path == 2:
            raise RuntimeError(self.lib.error())
        return size

    def project(self, x, codes, high, scales, out, workspace, available, *, tokens, n, k, padded, packed=False,
                stream=None):
        """Raw-pointer call of venturi_rowcodec_project (all arguments are device addresses or ints)."""
        return self.lib.check(
            self.lib.venturi_rowcodec_project(
                C.byref(self.raw), x, codes, high, scales, out, workspace, available, tokens, n, k, padded,
                int(packed), stream,
            )
        )


def prepare_row_codec(bits, group, *, precision="wxa16", dtype=0, implementation="auto", library=None):
    """Admits a plan or raises ValueError with the library's reason."""
    lib = native.load(library)
    raw = VRCPlan()
    if lib.venturi_rowcodec_prepare(bits, group, PRECISIONS[precision], dtype, IMPLEMENTATIONS[implementation],
                                    C.byref(raw)) != 0:
        raise ValueError(lib.error())
    return RowCodecPlan(lib, raw)
