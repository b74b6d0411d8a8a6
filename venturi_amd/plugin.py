"""Stand-alone row-codec operator objects over the library's plugin ABIs.

The reference ships two prebuilt operator objects with one shape of API,
``NativeQ4`` (ops/flash_next_q4.py:17-89, expert ABI 1) and ``NativeQ5``
(ops/flash_next_q5.py:17-89, Q5 ABI 1): ``prepare`` uploads a CPU descriptor
and records a ready event, ``decode`` returns the fp16 matrix of the contract
weights fp16(q * scale), ``linear`` runs the reference-order GEMV for 1..64
fp16 tokens, both allocating their output under an explicit byte budget. Here
one base class, ``RowCodecOperator``, carries that behaviour once, driven by a
``CodecEntry`` table row (descriptor type, plane names, ABI probe and the two
entry points); the codec classes only name their row. Qualification is gfx950
instead of SM70; error types and texts keep the reference's (with "GPU" for
"CUDA").
"""

from dataclasses import dataclass
from pathlib import Path

import torch


@dataclass(frozen=True)
class CodecEntry:
    label: str          # "Q4" / "Q5" in messages
    descriptor: type    # Q4RowSplitWeight / Q5RowSplitWeight
    planes: tuple       # descriptor fields passed to the kernels, in argument order
    abi: str            # ABI probe export; must return 1
    decode: str         # (planes..., out, rows, cols, padded, stream)
    linear: str         # (x, planes..., out, tokens, rows, cols, padded, stream)


class RowCodecOperator:
    """Shared body of the reference's plugin operators; subclasses set ``entry`` and ``prepared``."""

    entry: CodecEntry
    prepared: type
    max_tokens = 64

    def __init__(self, library=None, *, max_output_bytes=64 * 2**20):
        from . import native

        if type(max_output_bytes) is not int or max_output_bytes <= 0:
            raise ValueError("Positive explicit output budget required")
        self.max_output_bytes = max_output_bytes
        self.lib = native.load(library)
        self.library = Path(self.lib.path)
        if getattr(self.lib, self.entry.abi)() != 1:
            raise ValueError(f"Unsupported {self.entry.label} operator ABI")

    # -- helpers -------------------------------------------------------------
    def _within_budget(self, rows, cols):
        return rows * cols * 2 <= self.max_output_bytes

    def _planes(self, weight):
        return [getattr(weight, name) for name in self.entry.planes]

    def _claim(self, prepared):
        """Orders the current stream after the upload and ties the planes' lifetime to it."""
        label = self.entry.label
        if not isinstance(prepared, self.prepared) or prepared.weight.codes.device.type != "cuda":
            raise ValueError(f"Explicit prepared GPU {label} weight required")
        weight = prepared.weight
        weight.validate()
        stream = torch.cuda.current_stream(weight.codes.device)
        stream.wait_event(prepared.ready)
        for plane in self._planes(weight):
            plane.record_stream(stream)
        return weight, stream

    def _call(self, name, what, *arguments):
        status = getattr(self.lib, name)(*arguments)
        if status:
            raise RuntimeError(f"{self.entry.label} {what} HIP launch failed: {status}")

    # -- the reference's operator API --------------------------------------
    def prepare(self, weight, *, device):
        from .blocks import is_gfx950

        label = self.entry.label
        if not isinstance(weight, self.entry.descriptor) or weight.codes.device.type != "cpu":
            raise ValueError(f"Explicit CPU {label} descriptor required for preparation")
        weight.validate()
        scales = weight.scales
        admissible = bool(torch.isfinite(scales).all()) and not bool((scales < 0).any())
        if not (admissible and self._within_budget(weight.out_features, weight.in_features)):
            raise ValueError(f"Finite nonnegative {label} scales and bounded matrix required")
        target = torch.device(device)
        if target.type != "cuda":
            raise ValueError("Explicit GPU device required")
        with torch.cuda.device(target):
            if not is_gfx950(target):
                raise ValueError("This operator is qualified only for gfx950")
            resident = self.entry.descriptor(*(p.to(target) for p in self._planes(weight)), weight.in_features)
            ready = torch.cuda.Event()
            ready.record(torch.cuda.current_stream(target))
        return self.prepared(resident, ready)

    def decode(self, prepared):
        with torch.cuda.device(prepared.weight.codes.device):
            weight, stream = self._claim(prepared)
            rows, cols = weight.out_features, weight.in_features
            if not self._within_budget(rows, cols):
                raise ValueError(f"{self.entry.label} decode exceeds output budget")
            out = torch.empty((rows, cols), device=weight.codes.device, dtype=torch.float16)
            self._call(self.entry.decode, "decode", *(p.data_ptr() for p in self._planes(weight)), out.data_ptr(),
                       rows, cols, weight.padded_k, stream.cuda_stream)
            return out

    def linear(self, x, prepared):
        if not isinstance(prepared, self.prepared):
            raise ValueError(f"Explicit prepared GPU {self.entry.label} weight required")
        weight = prepared.weight
        fits = (
            isinstance(x, torch.Tensor) and x.ndim == 2 and 1 <= x.shape[0] <= self.max_tokens
            and x.shape[1] == weight.in_features and x.dtype == torch.float16
            and x.device == weight.codes.device and x.is_contiguous()
        )
        if not fits:
            raise ValueError("Bounded contiguous FP16 GPU input required")
        tokens = x.shape[0]
        if not self._within_budget(tokens, weight.out_features):
            raise ValueError(f"{self.entry.label} linear exceeds output budget")
        with torch.cuda.device(x.device):
            weight, stream = self._claim(prepared)
            out = torch.empty((tokens, weight.out_features), device=x.device, dtype=x.dtype)
            self._call(self.entry.linear, "GEMV", x.data_ptr(), *(p.data_ptr() for p in self._planes(weight)),
                       out.data_ptr(), tokens, weight.out_features, weight.in_features, weight.padded_k,
                       stream.cuda_stream)
            return out
