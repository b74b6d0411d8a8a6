"""Row-codec planes of one matrix in a standard .safetensors file.

The reference stores a quantized matrix with original name ``P`` and logical
shape [N, K] as separate tensors (docs/qwen-safetensors.md:45-58):

* ``P.codes``: int8 for Q8, uint8 otherwise, [N, groups * 32];
* ``P.high`` (Q5/Q6 only): uint8, [N, groups * 8 * (bits - 4)];
* ``P.scales``: float16, [N, groups];

with groups = padded_K / group (K padded to 128; group 32 for Q8, 64 for
Q4/Q5/Q6). The planes are exactly the row-split device layout, so they feed
the plan table (``RowCodecPlan.project``) and the resident-weight uploads
without any repacking. Admission follows the reference's loader: every plane
present with its exact shape and dtype (qwen_weights.py:58-92), Q8 without the
code -128, scales finite and not negative (qwen_weights.py:183-195). Plane
order in the file does not matter; each tensor is read by name.
"""

from dataclasses import dataclass
from typing import Optional

import torch

from .quantization.codecs import codec_for
from .quantization.layout import ROW_FORMATS
from .weights import Q4RowSplitWeight, Q5RowSplitWeight, Q8RowSplitWeight

_DTYPES = {"int8": torch.int8, "uint8": torch.uint8, "float16": torch.float16}
_SAFETENSORS_DTYPES = {"I8": "int8", "U8": "uint8", "F16": "float16"}


def plane_schema(name, fmt, shape):
    """The tensors a quantized matrix occupies: [(tensor name, shape, dtype name)]."""
    if fmt not in ROW_FORMATS:
        raise ValueError(f"not a row-codec format: {fmt!r}")
    n, k = (int(v) for v in shape)
    if n <= 0 or k <= 0:
        raise ValueError("matrix shape must be positive")
    codec = codec_for(fmt)
    groups = -(-k // 128) * 128 // codec.group
    schema = [(name + ".codes", (n, groups * 32), "int8" if codec.bits == 8 else "uint8")]
    if codec.high_plane:
        schema.append((name + ".high", (n, groups * 8 * (codec.bits - 4)), "uint8"))
    schema.append((name + ".scales", (n, groups), "float16"))
    return schema


@dataclass(frozen=True)
class MatrixPlanes:
    """Admitted CPU planes of one matrix (``high`` is None for Q8 and Q4)."""

    name: str
    fmt: str
    shape: tuple
    codes: torch.Tensor
    scales: torch.Tensor
    high: Optional[torch.Tensor] = None

    @property
    def padded_k(self):
        return -(-self.shape[1] // 128) * 128

    def weight(self):
        """The resident-weight descriptor over the same tensors (Q8, Q4 or Q5)."""
        k = self.shape[1]
        if self.fmt == "q8_g32_fp16":
            return Q8RowSplitWeight(self.codes, self.scales, k)
        if self.fmt == "q4_g64_fp16":
            return Q4RowSplitWeight(self.codes, self.scales, k)
        if self.fmt == "q5_g64_fp16":
            return Q5RowSplitWeight(self.codes, self.high, self.scales, k)
        raise ValueError(f"{self.fmt} has no resident-weight descriptor; project its planes through the plan table")


def _admit_values(fmt, codes, scales):
    scale = scales.float()
    if not bool(torch.isfinite(scale).all()) or bool((scale < 0).any()):
        raise ValueError("stored scales must be finite and nonnegative")
    if codec_for(fmt).bits == 8 and bool((codes == -128).any()):
        raise ValueError("Q8 planes may not hold the code -128")


def read_planes(path, name, fmt, shape):
    """Reads and admits the planes of matrix ``name`` ([N, K] logical shape, format ``fmt``).

    Raises ValueError for a missing plane, a plane of another shape or dtype,
    or stored values the format forbids.
    """
    from safetensors import safe_open

    schema = plane_schema(name, fmt, shape)
    tensors = {}
    with safe_open(str(path), framework="pt") as f:
        present = set(f.keys())
        for tensor, want_shape, want_dtype in schema:
            if tensor not in present:
                raise ValueError(f"missing plane: {tensor}")
            view = f.get_slice(tensor)
            dtype = _SAFETENSORS_DTYPES.get(view.get_dtype())
            if tuple(view.get_shape()) != want_shape or dtype != want_dtype:
                raise ValueError(f"plane shape/dtype mismatch: {tensor} holds {view.get_dtype()} "
                                 f"{tuple(view.get_shape())}, the format needs {want_dtype} {want_shape}")
            tensors[tensor[len(name) + 1:]] = f.get_tensor(tensor).contiguous()
    _admit_values(fmt, tensors["codes"], tensors["scales"])
    return MatrixPlanes(name, fmt, (int(shape[0]), int(shape[1])), tensors["codes"], tensors["scales"],
                        tensors.get("high"))


def planes_of(name, weight):
    """The named plane tensors of a Q8/Q4/Q5 weight, ready for ``safetensors.torch.save_file``."""
    if isinstance(weight, Q8RowSplitWeight) or isinstance(weight, Q4RowSplitWeight):
        planes = {name + ".codes": weight.codes, name + ".scales": weight.scales}
    elif isinstance(weight, Q5RowSplitWeight):
        planes = {name + ".codes": weight.codes, name + ".high": weight.high, name + ".scales": weight.scales}
    else:
        raise ValueError("planes_of takes a Q8, Q4 or Q5 row-split weight")
    for tensor, shape, dtype in plane_schema(name, weight.format, (weight.out_features, weight.in_features)):
        got = planes[tensor]
        if tuple(got.shape) != shape or got.dtype != _DTYPES[dtype]:
            raise ValueError(f"{tensor} does not match the stored schema")
    return {k: v.detach().cpu().contiguous() for k, v in planes.items()}
