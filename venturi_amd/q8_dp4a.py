"""W8A8 projection: int8 activations with fp32 group-32 scales, optional residual pass.

Mirrors venturi.ops.q8_dp4a (reference q8_dp4a.py:43-114): the plan quantizes
fp16 activations into a caller-owned workspace (``workspace_bytes`` bytes,
16-byte aligned, layout int8 codes [pass][token][group][32] then fp32 scales
[pass][token][group]) and projects them against the resident Q8 planes. Each
32-column group's integer dot is exact. Routes:

* ``exact``: groups combined in fp32 in the reference's lane-slot and
  shuffle-tree order (SIMT below 64 tokens, matrix cores above), so the fp16
  outputs are byte-identical to the reference's;
* ``mfma``: matrix cores with the scaled group terms summed in natural order
  (one accumulator per output), equal to the reference up to fp32
  association: up to 32 tokens the int8 decode kernel over the resident's
  tiled planes (``venturi_q8_a8_tiled_run``, the layout of the A16 decode
  route, built once per resident; ``run`` quantizes and projects in one
  launch through ``venturi_q8_a8_tiled_linear_run`` where the activations
  fit), above that the prefill GEMM's large tiles;
* ``auto``: ``mfma`` up to 32 tokens and from 64 (decode and prefill),
  ``exact`` between (the SIMT kernel streams the weights there, and the
  prefill GEMM's 256-token tiles would mostly hold padding).
"""

from dataclasses import dataclass

import torch

from .blocks import ResidentLinear
from .operands import admit, disjoint, extents, stream_of
from .vocabulary import ResidentQ8Vocabulary

A8_ROUTES = ("auto", "exact", "mfma")
A8_MFMA_MIN_AUTO_TOKENS = 64
A8_TILED_MAX_TOKENS = 32  # the int8 decode kernel's limit (two token blocks of 16)


@dataclass(frozen=True)
class PreparedQ8DP4A:
    resident: ResidentQ8Vocabulary
    tokens: int
    passes: int
    workspace_bytes: int
    _native: object
    kernel: str = "exact"
    slots: object = None  # exchange slots of a tiled launch that splits K (plan-owned, left idle by every run)

    @property
    def precision_profile(self):
        return "w8-a8-g32-f32scale" + ("-residual-a8" if self.passes == 2 else "")

    @property
    def route(self):
        return "venturi-q8-a8" if self.kernel == "exact" else "venturi-q8-a8-mfma"

    def quantize(self, x, *, workspace):
        """Only the activation quantization step (fills ``workspace``)."""
        r = self.resident
        admit(x, (self.tokens, r.hidden_size), torch.float16, r.device, "x")
        admit(workspace, (self.workspace_bytes,), torch.uint8, r.device, "workspace")
        disjoint(workspace, (x,) + r.storage_tensors)
        if workspace.data_ptr() % 16:
            raise ValueError("A8 workspace requires 16-byte alignment")
        with torch.cuda.device(r.device):
            r.backend._check(
                self._native.venturi_q8_dp4a_quantize(
                    x.data_ptr(), workspace.data_ptr(), self.workspace_bytes, self.tokens, r.hidden_size,
                    self.passes, stream_of(r.device),
                )
            )
        return workspace

    def project(self, *, out, workspace):
        """Only the int8 projection of an already filled workspace."""
        r = self.resident
        admit(out, (self.tokens, r.vocab_size), torch.float16, r.device, "out")
        admit(workspace, (self.workspace_bytes,), torch.uint8, r.device, "workspace")
        disjoint(out, (workspace,) + r.storage_tensors + self._slot_tensors)
        if workspace.data_ptr() % 16:
            raise ValueError("A8 workspace requires 16-byte alignment")
        tail = ()
        if self.kernel == "tiled":
            entry = self._native.venturi_q8_a8_tiled_run
            codes, scales = r.tiled_planes()
            tail = self._slot_args()
        else:
            entry = self._native.venturi_q8_dp4a_run if self.kernel == "exact" else self._native.venturi_q8_a8_gemm_run
            codes, scales = r.row_major_planes()
        with torch.cuda.device(r.device):
            r.backend._check(
                entry(
                    workspace.data_ptr(), self.workspace_bytes, codes.data_ptr(), scales.data_ptr(),
                    out.data_ptr(), self.tokens, r.vocab_size, r.hidden_size, r.padded_k, self.passes, *tail,
                    stream_of(r.device),
                )
            )
        return out

    @property
    def _slot_tensors(self):
        return () if self.slots is None else (self.slots,)

    def _slot_args(self):
        return (None, 0) if self.slots is None else (self.slots.data_ptr(), self.slots.numel())

    def run(self, x, *, out, workspace):
        r = self.resident
        admit(x, (self.tokens, r.hidden_size), torch.float16, r.device, "x")
        admit(out, (self.tokens, r.vocab_size), torch.float16, r.device, "out")
        admit(workspace, (self.workspace_bytes,), torch.uint8, r.device, "workspace")
        disjoint(out, (x, workspace) + r.storage_tensors + self._slot_tensors)
        disjoint(workspace, (x,) + r.storage_tensors + self._slot_tensors)
        if workspace.data_ptr() % 16:
            raise ValueError("A8 workspace requires 16-byte alignment")
        if self.kernel != "tiled":
            self.quantize(x, workspace=workspace)
            return self.project(out=out, workspace=workspace)
        codes, scales = r.tiled_planes()
        with torch.cuda.device(r.device):
            r.backend._check(
                self._native.venturi_q8_a8_tiled_linear_run(
                    x.data_ptr(), workspace.data_ptr(), self.workspace_bytes, codes.data_ptr(), scales.data_ptr(),
                    out.data_ptr(), self.tokens, r.vocab_size, r.hidden_size, r.padded_k, self.passes,
                    *self._slot_args(), stream_of(r.device),
                )
            )
        return out


def prepare_q8_dp4a(resident, *, tokens, residual_compensation, route="auto"):
    """Opt-in A8 plan; the caller owns the workspace (q8_dp4a.py:95-114).

    ``route`` (an addition to the reference's signature) selects the kernel
    family: "exact", "mfma" or "auto" (see the module docstring)."""
    if route not in A8_ROUTES:
        raise ValueError(f"A8 route must be one of {A8_ROUTES}")
    if isinstance(resident, ResidentLinear):
        resident = resident._payload
    if not isinstance(resident, ResidentQ8Vocabulary):
        raise ValueError("A8 requires resident native Q8 planes")
    resident.row_major_planes()  # the A8 kernels read the row-major planes
    if type(residual_compensation) is not bool:
        raise ValueError("Explicit boolean residual_compensation required")
    extents(tokens, resident.hidden_size)
    if resident.dtype != torch.float16 or resident.device.type != "cuda":
        raise ValueError("A8 profile requires GPU FP16 input/output")
    resident.backend.validate_device(resident.dtype, resident.device)
    if tokens * resident.vocab_size >= 2**31:
        raise ValueError("A8 output geometry exceeds int32")
    native = resident.backend._native
    passes = 2 if residual_compensation else 1
    size = native.venturi_q8_dp4a_bytes(tokens, resident.hidden_size, passes)
    if not size:
        resident.backend._check(-1)
    if route == "auto":
        route = "mfma" if tokens >= A8_MFMA_MIN_AUTO_TOKENS or tokens <= A8_TILED_MAX_TOKENS else "exact"
    kernel = route
    if route == "mfma" and tokens <= A8_TILED_MAX_TOKENS:
        kernel = "tiled"
        resident.tiled_planes()  # built once per resident, outside any capture
        slots = _a8_slots(resident, tokens, passes)
        return PreparedQ8DP4A(resident, tokens, passes, size, native, kernel, slots)
    return PreparedQ8DP4A(resident, tokens, passes, size, native, kernel)


def _a8_slots(resident, tokens, passes):
    """The plan's exchange slots when its tiled launch splits K (None when it does not).

    Every run leaves them idle again, so runs of one plan must be ordered (one
    stream at a time); concurrent streams prepare a plan each."""
    lib = resident.backend._native
    nbytes = lib.venturi_q8_a8_tiled_workspace_bytes(tokens, resident.vocab_size, resident.hidden_size, passes)
    if nbytes == 0:
        resident.backend._check(-1 if lib.venturi_blocks_error() else 0)
        return None
    with torch.cuda.device(resident.device):
        slots = torch.empty(nbytes, dtype=torch.uint8, device=resident.device)
        resident.backend._check(lib.venturi_q8_tiled_workspace_init(slots.data_ptr(), nbytes, stream_of(resident.device)))
        torch.cuda.current_stream(resident.device).synchronize()
    return slots
