"""Resident Q8 row-split planes: projection (output head) and embedding lookup.

Mirrors venturi.ops.vocabulary (reference vocabulary.py:23-173). A resident
Q8 matrix keeps its int8 codes and fp16 group scales on the device and is
never expanded to dense weights. ``prepare(tokens=...)`` selects the kernel
family once:

* ``exact``: the reference's canonical fp32 order (bytes identical to
  ``venturi_q8_head_run`` on the reference's GPUs);
* ``mfma``: fp16 matrix cores with per-group fp32 scaling (same values up to
  fp32 association, see ``Q8OutputHead.route``). Up to 32 tokens (decode)
  it reads a tiled copy of the planes (16-row blocks x 64-column chunks in
  MFMA operand order, built once by the first such plan and kept with the
  resident weight), so every wave streams contiguous 1 KB blocks; above 32
  tokens (prefill) it runs ``venturi_q8_prefill_run`` on the row-major planes
  (LDS-staged 256-token x 128-row tiles);
* ``auto``: ``mfma`` whenever its conditions hold (FP16 activations,
  K % 8 == 0), else ``exact``. The matrix-core kernels are faster at every
  token count (the canonical order needs one fp32 FMA per token and weight
  plus an exact weight conversion, and its lane-per-four-columns layout
  issues 4-byte loads); callers that need the reference's bytes ask for
  ``exact``.
"""

from dataclasses import dataclass, field
import threading

import torch

from .blocks import _DTYPES, Q8_ROUTES, _no_overlap, _shape, _stream, _tensor

EXACT_MAX_AUTO_TOKENS = 0
MFMA_MAX_TOKENS = 32
_TILE_LOCK = threading.Lock()


def tile_q8(codes, scales, paired=False):
    """Tiled planes of the matrix-core route (read by ``venturi_q8_tiled_run``).

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
        idx = torch.arange(blocks * 16, device=codes.device)
        gate = (idx // 16) * 8 + idx % 8  # intermediate column of each slot
        source = torch.where(idx % 16 < 8, gate, gate + inter)
        valid = gate < inter
        c = torch.zeros((blocks * 16, padded), dtype=torch.int8, device=codes.device)
        s = torch.zeros((blocks * 16, padded // 32), dtype=torch.float16, device=codes.device)
        c[valid] = codes[source[valid]]
        s[valid] = scales[source[valid]]
    else:
        blocks = (n + 15) // 16
        c = torch.zeros((blocks * 16, padded), dtype=torch.int8, device=codes.device)
        s = torch.zeros((blocks * 16, padded // 32), dtype=torch.float16, device=codes.device)
        c[:n] = codes
        s[:n] = scales
    tc = c.view(blocks, 16, chunks, 2, 4, 8).permute(0, 2, 4, 1, 3, 5).contiguous()
    ts = s.view(blocks, 16, chunks, 2).permute(0, 2, 1, 3).contiguous()
    return tc, ts


def _ids(ids, vocab):
    if not isinstance(ids, (list, tuple)) or not ids:
        raise ValueError("Vocabulary IDs must be a nonempty list/tuple")
    if len(ids) >= 2**31 or any(type(i) is not int or not 0 <= i < vocab for i in ids):
        raise ValueError("Vocabulary ID/count is out of range")


@dataclass(frozen=True)
class Q8VocabularyWeights:
    codes: torch.Tensor
    scales: torch.Tensor
    hidden_size: int

    def validate(self):
        if type(self.hidden_size) is not int or self.hidden_size <= 0:
            raise ValueError("Q8 hidden size must be positive")
        if not isinstance(self.codes, torch.Tensor) or self.codes.ndim != 2:
            raise ValueError("Q8 codes require [vocab,padded_hidden]")
        n, padded = self.codes.shape
        _shape(n, self.hidden_size)
        if padded != (self.hidden_size + 127) // 128 * 128:
            raise ValueError("Q8 hidden padding must be a multiple of 128")
        device = self.codes.device
        _tensor(self.codes, (n, padded), torch.int8, device, "codes")
        _tensor(self.scales, (n, padded // 32), torch.float16, device, "scales")
        if bool((self.codes == -128).any()):
            raise ValueError("Q8 code -128 is outside the artifact contract")
        if not bool(torch.isfinite(self.scales).all()) or bool((self.scales < 0).any()):
            raise ValueError("Q8 scales must be finite and nonnegative")

    def upload(self, backend, *, device="cuda:0", dtype=torch.bfloat16):
        """Copies the planes to the device once (a same-device source is copied too)."""
        self.validate()
        if dtype not in (torch.float16, torch.bfloat16):
            raise ValueError("Q8 vocabulary supports FP16/BF16 activations")
        target = backend.validate_device(dtype, device)
        with torch.cuda.device(target):
            codes, scales = (t.detach().to(target, copy=True) for t in (self.codes, self.scales))
            torch.cuda.current_stream(target).synchronize()
        return ResidentQ8Vocabulary(backend, codes, scales, self.hidden_size, dtype)


@dataclass(frozen=True)
class ResidentQ8Vocabulary:
    backend: object
    _codes: torch.Tensor
    _scales: torch.Tensor
    hidden_size: int
    dtype: torch.dtype = torch.bfloat16
    _tiles: dict = field(default_factory=dict, compare=False, repr=False)

    @property
    def device(self):
        return self._codes.device

    def tiled_planes(self, paired=False):
        """The matrix-core route's tiled copy of the planes (built on first use)."""
        key = "mfma-paired" if paired else "mfma"
        with _TILE_LOCK:
            if key not in self._tiles:
                with torch.cuda.device(self.device):
                    self._tiles[key] = tile_q8(self._codes, self._scales, paired)
                    torch.cuda.current_stream(self.device).synchronize()
            return self._tiles[key]

    @property
    def vocab_size(self):
        return self._codes.shape[0]

    @property
    def storage_tensors(self):
        return (self._codes, self._scales)

    @property
    def storage_nbytes(self):
        return sum(t.numel() * t.element_size() for t in self.storage_tensors)

    def prepare_embedding(self, ids):
        _ids(ids, self.vocab_size)
        self.backend.validate_device(self.dtype, self.device)
        indices = torch.tensor(ids, dtype=torch.int64, device=self.device)
        torch.cuda.current_stream(self.device).synchronize()
        return Q8Embedding(self, indices)

    def prepare(self, *, tokens, route="auto"):
        _shape(tokens, self.vocab_size)
        if tokens * self.vocab_size >= 2**31:
            raise ValueError("Q8 head row count must fit int32")
        if route not in Q8_ROUTES:
            raise ValueError(f"Q8 route must be one of {Q8_ROUTES}")
        self.backend.validate_device(self.dtype, self.device)
        mfma_ok = self.dtype == torch.float16 and self.hidden_size % 8 == 0
        if route == "auto":
            route = "mfma" if mfma_ok and tokens > EXACT_MAX_AUTO_TOKENS else "exact"
        if route == "mfma" and not mfma_ok:
            raise ValueError("The Q8 MFMA route takes FP16 activations and K % 8 == 0")
        if route == "exact":
            return Q8OutputHead(self, tokens, route)
        if tokens > MFMA_MAX_TOKENS:
            return Q8OutputHead(self, tokens, "prefill")
        return Q8OutputHead(self, tokens, route, self.tiled_planes(), self._slots(tokens, swiglu=False))

    def _slots(self, tokens, *, swiglu):
        """The plan's exchange slots for launches that split K (None when this shape does not split)."""
        lib = self.backend._native
        nbytes = lib.venturi_q8_tiled_workspace_bytes(tokens, self.vocab_size, int(swiglu))
        if nbytes == 0:
            self.backend._check(-1 if lib.venturi_blocks_error() else 0)
            return None
        with torch.cuda.device(self.device):
            slots = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
            self.backend._check(lib.venturi_q8_tiled_workspace_init(slots.data_ptr(), nbytes, _stream(self.device)))
            torch.cuda.current_stream(self.device).synchronize()
        return slots


    def prepare_swiglu(self, *, tokens):
        """Fused gate+up projection with SwiGLU (an extension; matrix cores only).

        The resident matrix is [2 * inter, hidden] with the gate rows first; the
        plan writes out [tokens, inter] = fp16(swiglu(fp16(gate), fp16(up))), the
        bytes of the ``mfma`` projection followed by ``venturi_silu_mul_run``.
        """
        _shape(tokens, self.vocab_size)
        if self.vocab_size % 2:
            raise ValueError("a fused gate+up matrix needs an even row count")
        if not (self.dtype == torch.float16 and self.hidden_size % 8 == 0 and tokens <= MFMA_MAX_TOKENS):
            raise ValueError(
                f"The fused SwiGLU projection takes FP16 activations, K % 8 == 0 and at most {MFMA_MAX_TOKENS} tokens"
            )
        self.backend.validate_device(self.dtype, self.device)
        return Q8OutputHead(self, tokens, "swiglu", self.tiled_planes(paired=True), self._slots(tokens, swiglu=True))


@dataclass(frozen=True)
class Q8Embedding:
    resident: ResidentQ8Vocabulary
    _indices: torch.Tensor

    def run(self, *, out):
        r = self.resident
        _tensor(out, (self._indices.numel(), r.hidden_size), r.dtype, r.device, "out")
        _no_overlap(out, r.storage_tensors + (self._indices,))
        with torch.cuda.device(r.device):
            r.backend._check(
                r.backend._native.venturi_q8_embedding_run(
                    r._codes.data_ptr(),
                    r._scales.data_ptr(),
                    self._indices.data_ptr(),
                    out.data_ptr(),
                    self._indices.numel(),
                    r.vocab_size,
                    r.hidden_size,
                    r._codes.shape[1],
                    _DTYPES[r.dtype],
                    _stream(r.device),
                )
            )
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
    workspace_bytes = 0

    @property
    def route(self):
        return {
            "exact": "venturi-q8-exact",
            "mfma": "venturi-q8-mfma",
            "prefill": "venturi-q8-mfma",
            "swiglu": "venturi-q8-mfma-swiglu",
        }[self.kernel]

    @property
    def out_features(self):
        n = self.resident.vocab_size
        return n // 2 if self.kernel == "swiglu" else n

    @property
    def storage_tensors(self):
        return self.resident.storage_tensors + tuple(self.tiles)

    def run(self, x, *, out):
        r = self.resident
        _tensor(x, (self.tokens, r.hidden_size), r.dtype, r.device, "x")
        _tensor(out, (self.tokens, self.out_features), r.dtype, r.device, "out")
        slots = () if self.slots is None else (self.slots,)
        _no_overlap(out, (x,) + self.storage_tensors + slots)
        lib = r.backend._native
        if self.kernel == "exact":
            entry, planes, tail = lib.venturi_q8_head_run, (r._codes, r._scales), ()
        elif self.kernel == "prefill":
            entry, planes, tail = lib.venturi_q8_prefill_run, (r._codes, r._scales), ()
        else:
            entry = lib.venturi_q8_tiled_swiglu_run if self.kernel == "swiglu" else lib.venturi_q8_tiled_run
            planes = self.tiles
            tail = (0, 0) if self.slots is None else (self.slots.data_ptr(), self.slots.numel())
        with torch.cuda.device(r.device):
            r.backend._check(
                entry(
                    x.data_ptr(),
                    planes[0].data_ptr(),
                    planes[1].data_ptr(),
                    out.data_ptr(),
                    self.tokens,
                    r.vocab_size,
                    r.hidden_size,
                    r._codes.shape[1],
                    _DTYPES[r.dtype],
                    *tail,
                    _stream(r.device),
                )
            )
        return out
