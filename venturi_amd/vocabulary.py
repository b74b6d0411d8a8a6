"""Resident Q8 row-split matrices: output projection (the vocabulary head) and embedding lookup.

Public names of the reference's ops/vocabulary.py (lines 23-173):
``Q8VocabularyWeights(codes, scales, hidden_size)`` with ``validate`` and
``upload``; ``ResidentQ8Vocabulary`` with ``prepare(tokens=)``,
``prepare_embedding(ids)``, ``storage_tensors``; ``Q8OutputHead.run(x, out=)``
and ``Q8Embedding.run(out=)``. The matrix is never expanded to dense weights.

Kernel families, chosen once per plan (``prepare(tokens=, route=)``):

* ``exact``: the reference's canonical fp32 order (``venturi_q8_head_run``,
  the bytes of the reference's head kernel), row-major planes;
* ``mfma``: fp16 matrix cores with per-group fp32 scaling (equal to the
  canonical order up to fp32 association). Up to 32 tokens (decode) it reads
  the tiled planes (16-row blocks x 64-column chunks in MFMA operand order),
  so each wave streams contiguous 1 KB blocks; above 32 tokens (prefill) it
  runs ``venturi_q8_prefill_run`` on the row-major planes;
* ``dense``: for prefill, each chunk of rows decoded to the exact two-term
  fp16 form of its weights (q*s = hi + lo, ``venturi_q8_dense_run``) and
  multiplied by hipBLASLt over the doubled K (every product exact, fp32
  sums: equal to the canonical order up to fp32 association); FP16, K and N
  multiples of 8, row-major planes, every scale below 516; the plan takes a
  caller-owned workspace of ``workspace_bytes`` (the two-term fp16 shadow of
  a chunk of up to 8192 rows, 4 bytes per weight, plus hipBLASLt's 32 MiB:
  210-533 MB at the config-2 shapes);
  ``run(x, out=)`` without one, as the reference calls a plan, runs the
  ``mfma`` prefill kernel instead (no workspace, the same tolerance);
* ``auto``: ``dense`` from DENSE_TOKENS tokens where its conditions hold,
  else ``mfma`` where its conditions hold (FP16 activations, K % 8 == 0),
  else ``exact``.

Residency (an upload option): ``"row-major"`` keeps the planes as the
reference lays them out and builds a tiled copy the first time a decode plan
needs it (both stay resident: 2.1 bytes per weight); ``"tiled"`` keeps only
the tiled copy (1.06 bytes per weight) and admits decode plans of at most 32
tokens on the matrix-core route; ``"tiled-paired"`` keeps only the paired
copy of a gate+up matrix and admits ``prepare_swiglu``. The single-copy forms
suit large matrices that only decode reads, such as a 248 320-row head.
"""

from dataclasses import dataclass, field
import threading

import torch

from .blocks import Q8_ROUTES
from .operands import DTYPE_CODES, admit, disjoint, extents, stream_of

EXACT_MAX_AUTO_TOKENS = 0
MFMA_MAX_TOKENS = 32
# The dense route decodes and writes 4 bytes per weight before its GEMM, so it
# pays only at large token counts: config-2 shapes against the fused GEMM at
# 1024 tokens 0.87-1.28x (gate+up and down slower), at 2048 1.13-1.21x.
DENSE_TOKENS = 2048
DENSE_MAX_SCALE = 516.0  # 127 * 516 rounds past the fp16 range
RESIDENCIES = ("row-major", "tiled", "tiled-paired")
_TILE_LOCK = threading.Lock()
_ROUTE_NAMES = {"exact": "venturi-q8-exact", "mfma": "venturi-q8-mfma", "prefill": "venturi-q8-mfma",
                "swiglu": "venturi-q8-mfma-swiglu", "dense": "venturi-q8-dense"}


def _padded(k):
    return (k + 127) // 128 * 128


def tile_q8(codes, scales, paired=False):
    """Tiled planes of the matrix-core decode (read by ``venturi_q8_tiled_run``).

    Codes [row block][chunk][lane l = 16q + m][16 bytes]: row m of the block,
    columns 64c + 8q .. +8 (group 2c) then 64c + 32 + 8q .. +8 (group 2c + 1).
    Scales [row block][chunk][m][2] fp16. Rows are padded to a multiple of 16
    with zero codes and scales. ``paired`` (a fused gate+up matrix, gate rows
    first, read by ``venturi_q8_tiled_swiglu_run``): block b holds gate rows
    8b..8b+7 in slots 0..7 and the matching up rows in slots 8..15.
    """
    n, padded = codes.shape
    chunks = padded // 64
    if paired:
        if n % 2:
            raise ValueError("a fused gate+up matrix needs an even row count")
        inter = n // 2
        blocks = (inter + 7) // 8
        slot = torch.arange(blocks * 16, device=codes.device)
        column = (slot // 16) * 8 + slot % 8  # the intermediate column each slot serves
        source = torch.where(slot % 16 < 8, column, column + inter)
        keep = column < inter
    else:
        blocks = (n + 15) // 16
        source = torch.arange(blocks * 16, device=codes.device)
        keep = source < n
    c = torch.zeros((blocks * 16, padded), dtype=torch.int8, device=codes.device)
    s = torch.zeros((blocks * 16, padded // 32), dtype=torch.float16, device=codes.device)
    c[keep] = codes[source[keep]]
    s[keep] = scales[source[keep]]
    tiled_codes = c.view(blocks, 16, chunks, 2, 4, 8).permute(0, 2, 4, 1, 3, 5).contiguous()
    tiled_scales = s.view(blocks, 16, chunks, 2).permute(0, 2, 1, 3).contiguous()
    return tiled_codes, tiled_scales


def _ids(ids, vocab):
    if not isinstance(ids, (list, tuple)) or not ids:
        raise ValueError("Vocabulary IDs must be a nonempty list/tuple")
    if len(ids) >= 2**31 or not all(type(i) is int and 0 <= i < vocab for i in ids):
        raise ValueError("Vocabulary ID/count is out of range")


@dataclass(frozen=True)
class Q8VocabularyWeights:
    """Q8 planes of one matrix (CPU or device): codes int8 [N, Kp], scales fp16 [N, Kp/32]."""

    codes: torch.Tensor
    scales: torch.Tensor
    hidden_size: int

    def validate(self):
        if type(self.hidden_size) is not int or self.hidden_size <= 0:
            raise ValueError("Q8 hidden size must be positive")
        if not isinstance(self.codes, torch.Tensor) or self.codes.ndim != 2:
            raise ValueError("Q8 codes require [vocab,padded_hidden]")
        rows, width = self.codes.shape
        extents(rows, self.hidden_size)
        if width != _padded(self.hidden_size):
            raise ValueError("Q8 hidden padding must be a multiple of 128")
        where = self.codes.device
        admit(self.codes, (rows, width), torch.int8, where, "codes")
        admit(self.scales, (rows, width // 32), torch.float16, where, "scales")
        if bool((self.codes == -128).any()):
            raise ValueError("Q8 code -128 is outside the artifact contract")
        if bool((self.scales < 0).any()) or not bool(torch.isfinite(self.scales).all()):
            raise ValueError("Q8 scales must be finite and nonnegative")

    def upload(self, backend, *, device="cuda:0", dtype=torch.bfloat16, residency="row-major"):
        """Copies the planes to the device once (a same-device source is copied too).

        ``residency`` selects what stays resident (see the module docstring);
        the single-copy forms are built from a transient device copy.
        """
        self.validate()
        if dtype not in (torch.float16, torch.bfloat16):
            raise ValueError("Q8 vocabulary supports FP16/BF16 activations")
        if residency not in RESIDENCIES:
            raise ValueError(f"Q8 residency must be one of {RESIDENCIES}")
        target = backend.validate_device(dtype, device)
        geometry = (self.codes.shape[0], self.codes.shape[1])
        with torch.cuda.device(target):
            planes = tuple(t.detach().to(target, copy=True) for t in (self.codes, self.scales))
            tiles = {}
            if residency != "row-major":
                if dtype != torch.float16 or self.hidden_size % 8:
                    raise ValueError("tiled residency serves the matrix-core route: FP16 activations and K % 8 == 0")
                paired = residency == "tiled-paired"
                tiles[residency] = tile_q8(*planes, paired=paired)
                planes = (None, None)
            torch.cuda.current_stream(target).synchronize()
        return ResidentQ8Vocabulary(backend, planes[0], planes[1], self.hidden_size, dtype, tiles, residency,
                                    geometry, target)


@dataclass(frozen=True)
class ResidentQ8Vocabulary:
    backend: object
    _codes: object  # int8 [N, Kp] on the device, or None when only tiled planes are resident
    _scales: object
    hidden_size: int
    dtype: torch.dtype = torch.bfloat16
    _tiles: dict = field(default_factory=dict, compare=False, repr=False)
    residency: str = "row-major"
    _geometry: tuple = ()  # (rows, padded K)
    _device: object = None
    _facts: dict = field(default_factory=dict, compare=False, repr=False)  # cached plane properties

    @property
    def device(self):
        return self._device if self._device is not None else self._codes.device

    @property
    def vocab_size(self):
        return self._geometry[0] if self._geometry else self._codes.shape[0]

    @property
    def padded_k(self):
        return self._geometry[1] if self._geometry else self._codes.shape[1]

    @property
    def storage_tensors(self):
        if self.residency == "row-major":
            return (self._codes, self._scales)
        return self._tiles[self.residency]

    @property
    def storage_nbytes(self):
        return sum(t.numel() * t.element_size() for t in self.storage_tensors)

    def row_major_planes(self):
        """(codes, scales) of the reference layout; residents without them refuse clearly."""
        if self._codes is None:
            raise ValueError(f"this Q8 resident keeps only tiled planes (residency={self.residency!r}); "
                             "upload it with residency='row-major' for this kernel")
        return self._codes, self._scales

    def dense_admissible(self):
        """Whether the dense route's two-term form is exact for these planes
        (row-major planes kept, every scale below DENSE_MAX_SCALE); computed once."""
        if self._codes is None:
            return False
        with _TILE_LOCK:
            if "dense" not in self._facts:
                with torch.cuda.device(self.device):
                    self._facts["dense"] = bool((self._scales.float().abs() < DENSE_MAX_SCALE).all())
            return self._facts["dense"]

    def tiled_planes(self, paired=False):
        """The tiled copy of the planes (built on first use for a row-major resident)."""
        key = "tiled-paired" if paired else "tiled"
        with _TILE_LOCK:
            if key not in self._tiles:
                codes, scales = self.row_major_planes()
                with torch.cuda.device(self.device):
                    self._tiles[key] = tile_q8(codes, scales, paired)
                    torch.cuda.current_stream(self.device).synchronize()
            return self._tiles[key]

    def prepare_embedding(self, ids):
        _ids(ids, self.vocab_size)
        self.row_major_planes()
        self.backend.validate_device(self.dtype, self.device)
        indices = torch.tensor(ids, dtype=torch.int64, device=self.device)
        torch.cuda.current_stream(self.device).synchronize()
        return Q8Embedding(self, indices)

    def prepare(self, *, tokens, route="auto"):
        extents(tokens, self.vocab_size)
        if tokens * self.vocab_size >= 2**31:
            raise ValueError("Q8 head row count must fit int32")
        if route not in Q8_ROUTES:
            raise ValueError(f"Q8 route must be one of {Q8_ROUTES}")
        self.backend.validate_device(self.dtype, self.device)
        matrix_cores = self.dtype == torch.float16 and self.hidden_size % 8 == 0
        dense_shape = matrix_cores and self.vocab_size % 8 == 0 and tokens <= 65535
        if route == "auto":
            if dense_shape and tokens >= DENSE_TOKENS and self.dense_admissible():
                route = "dense"
            else:
                route = "mfma" if matrix_cores and tokens > EXACT_MAX_AUTO_TOKENS else "exact"
        if route == "mfma" and not matrix_cores:
            raise ValueError("The Q8 MFMA route takes FP16 activations and K % 8 == 0")
        if route == "dense":
            if not dense_shape:
                raise ValueError("The dense Q8 route takes FP16 activations, K and N multiples of 8, <= 65535 tokens")
            self.row_major_planes()
            if not self.dense_admissible():
                raise ValueError(f"The dense Q8 route needs every scale below {DENSE_MAX_SCALE}")
            lib = self.backend._native
            size = int(lib.venturi_q8_dense_workspace_bytes(tokens, self.vocab_size, self.hidden_size))
            if size == 0:
                raise ValueError(lib.error())
            return Q8OutputHead(self, tokens, "dense", workspace_bytes=size)
        if self.residency == "tiled-paired" or (self.residency == "tiled" and (route == "exact" or tokens > MFMA_MAX_TOKENS)):
            self.row_major_planes()  # raises: the plan needs planes this resident does not keep
        if route == "exact":
            return Q8OutputHead(self, tokens, "exact")
        if tokens > MFMA_MAX_TOKENS:
            return Q8OutputHead(self, tokens, "prefill")
        return Q8OutputHead(self, tokens, "mfma", self.tiled_planes(), self._slots(tokens, swiglu=False))

    def prepare_swiglu(self, *, tokens):
        """Fused gate+up projection with SwiGLU (an extension; matrix cores only).

        The resident matrix is [2 * inter, hidden] with the gate rows first; the
        plan writes out [tokens, inter] = fp16(swiglu(fp16(gate), fp16(up))), the
        bytes of the ``mfma`` projection followed by ``venturi_silu_mul_run``.
        """
        extents(tokens, self.vocab_size)
        if self.vocab_size % 2:
            raise ValueError("a fused gate+up matrix needs an even row count")
        if not (self.dtype == torch.float16 and self.hidden_size % 8 == 0 and tokens <= MFMA_MAX_TOKENS):
            raise ValueError(
                f"The fused SwiGLU projection takes FP16 activations, K % 8 == 0 and at most {MFMA_MAX_TOKENS} tokens"
            )
        if self.residency == "tiled":
            self.row_major_planes()
        self.backend.validate_device(self.dtype, self.device)
        return Q8OutputHead(self, tokens, "swiglu", self.tiled_planes(paired=True), self._slots(tokens, swiglu=True))

    def _slots(self, tokens, *, swiglu):
        """The plan's exchange slots for launches that split K (None when this shape does not split)."""
        lib = self.backend._native
        nbytes = lib.venturi_q8_tiled_workspace_bytes(tokens, self.vocab_size, int(swiglu))
        if nbytes == 0:
            self.backend._check(-1 if lib.venturi_blocks_error() else 0)
            return None
        with torch.cuda.device(self.device):
            slots = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
            self.backend._check(lib.venturi_q8_tiled_workspace_init(slots.data_ptr(), nbytes, stream_of(self.device)))
            torch.cuda.current_stream(self.device).synchronize()
        return slots


@dataclass(frozen=True)
class Q8Embedding:
    resident: ResidentQ8Vocabulary
    _indices: torch.Tensor

    def run(self, *, out):
        r = self.resident
        codes, scales = r.row_major_planes()
        admit(out, (self._indices.numel(), r.hidden_size), r.dtype, r.device, "out")
        disjoint(out, (codes, scales, self._indices))
        with torch.cuda.device(r.device):
            r.backend._check(r.backend._native.venturi_q8_embedding_run(
                codes.data_ptr(), scales.data_ptr(), self._indices.data_ptr(), out.data_ptr(), self._indices.numel(),
                r.vocab_size, r.hidden_size, r.padded_k, DTYPE_CODES[r.dtype], stream_of(r.device)))
        return out


@dataclass(frozen=True)
class Q8OutputHead:
    """A prepared projection. Matrix-core plans whose launch splits K over two
    workgroups own an exchange-slot buffer that every run leaves idle again;
    runs of one such plan must therefore be ordered (one stream at a time)."""

    resident: ResidentQ8Vocabulary
    tokens: int
    kernel: str = "exact"
    tiles: tuple = ()
    slots: object = None
    workspace_bytes: int = 0  # the dense route's caller-owned workspace

    @property
    def route(self):
        return _ROUTE_NAMES[self.kernel]

    @property
    def out_features(self):
        n = self.resident.vocab_size
        return n // 2 if self.kernel == "swiglu" else n

    @property
    def storage_tensors(self):
        r = self.resident
        kept = () if r._codes is None else (r._codes, r._scales)
        return kept + tuple(self.tiles) + (() if self.slots is None else (self.slots,))

    def run(self, x, *, out, workspace=None):
        r = self.resident
        if self.kernel != "dense" and workspace is not None:
            raise ValueError("This Q8 plan uses no workspace")
        admit(x, (self.tokens, r.hidden_size), r.dtype, r.device, "x")
        admit(out, (self.tokens, self.out_features), r.dtype, r.device, "out")
        disjoint(out, (x,) + self.storage_tensors)
        lib = r.backend._native
        kernel = self.kernel
        if kernel == "dense" and workspace is None:
            # The reference's run(x, out=) passes no workspace: the fused
            # matrix-core prefill kernel, which needs none, serves the call.
            kernel = "prefill"
        if kernel == "dense":
            admit(workspace, (self.workspace_bytes,), torch.uint8, r.device, "workspace")
            if workspace.data_ptr() % 256 or x.data_ptr() % 16 or out.data_ptr() % 16:
                raise ValueError("the dense Q8 route needs a 256-byte aligned workspace and 16-byte aligned x and out")
            disjoint(workspace, (x, out) + self.storage_tensors)
            codes, scales = r.row_major_planes()
            with torch.cuda.device(r.device):
                r.backend._check(lib.venturi_q8_dense_run(
                    x.data_ptr(), codes.data_ptr(), scales.data_ptr(), out.data_ptr(), self.tokens, r.vocab_size,
                    r.hidden_size, r.padded_k, DTYPE_CODES[r.dtype], workspace.data_ptr(), self.workspace_bytes,
                    stream_of(r.device)))
            return out
        if kernel in ("exact", "prefill"):
            entry = lib.venturi_q8_head_run if kernel == "exact" else lib.venturi_q8_prefill_run
            planes, tail = r.row_major_planes(), ()
        else:
            entry = lib.venturi_q8_tiled_swiglu_run if kernel == "swiglu" else lib.venturi_q8_tiled_run
            planes = self.tiles
            tail = (0, 0) if self.slots is None else (self.slots.data_ptr(), self.slots.numel())
        with torch.cuda.device(r.device):
            r.backend._check(entry(x.data_ptr(), planes[0].data_ptr(), planes[1].data_ptr(), out.data_ptr(),
                                   self.tokens, r.vocab_size, r.hidden_size, r.padded_k, DTYPE_CODES[r.dtype], *tail,
                                   stream_of(r.device)))
        return out
