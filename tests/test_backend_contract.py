"""The prepared-operator contract on the host (no GPU, no library load): capability
records, exact format/layout matching, validation errors and the factory's
refusal to fall back, as the reference's contract tests check them
(tests/test_backend_contract.py:45-140)."""

from dataclasses import FrozenInstanceError

import pytest
import torch

from venturi_amd.backend import (
    Backend,
    BackendCapabilities,
    OperatorSupport,
    UnsupportedOperationError,
    create_backend,
)
from venturi_amd.blocks import HipBackend


@pytest.mark.parametrize("kind", ["auto", "metal", "mlx", "mps", "unknown", None])
def test_unknown_backend_kind_is_not_a_silent_fallback(kind):
    with pytest.raises(UnsupportedOperationError, match="not implemented"):
        create_backend(kind)


def test_torch_backend_is_refused_explicitly():
    with pytest.raises(UnsupportedOperationError, match="not part of venturi_amd"):
        create_backend("torch")


def test_hip_capabilities_match_format_and_layout_exactly():
    caps = object.__new__(HipBackend).capabilities  # metadata only: no library load
    assert caps.cuda_graphs and not caps.reference
    for fmt in ("q4_g64_fp16", "q8_g32_fp16"):
        assert caps.supports("linear", dtype=torch.float16, device="cuda:3", weight_format=fmt,
                             weight_layout="row_split_k128_v1")
        for layout in (None, "gptq", "row_split_k256_v9"):
            assert not caps.supports("linear", dtype=torch.float16, device="cuda:0", weight_format=fmt,
                                     weight_layout=layout)
    assert caps.supports("embedding", dtype=torch.bfloat16, device="cuda", weight_format="q8_g32_fp16",
                         weight_layout="row_split_k128_v1")
    assert not caps.supports("embedding", dtype=torch.float16, device="cuda", weight_format="q4_g64_fp16",
                             weight_layout="row_split_k128_v1")
    assert caps.supports("rmsnorm", dtype=torch.float32, device="cuda:1")
    assert not caps.supports("linear", dtype=torch.float16, device="cpu", weight_format="q8_g32_fp16",
                             weight_layout="row_split_k128_v1")
    assert not caps.supports("linear", dtype=torch.float16, device="cuda")  # dense weights are not declared
    assert not caps.supports("moe", dtype=torch.float16, device="cuda")
    with pytest.raises(FrozenInstanceError):
        caps.cuda_graphs = False
    with pytest.raises(UnsupportedOperationError, match="no automatic fallback"):
        caps.require("linear", dtype=torch.float32, device="cuda", weight_format="q8_g32_fp16",
                     weight_layout="row_split_k128_v1")


def test_operator_support_snapshots_its_sets():
    """A capability record keeps what it was given at construction: later changes to the caller's
    device and dtype sets do not reach it (reference contract, tests/test_backend_contract.py)."""
    devices, dtypes = {"cpu"}, {torch.float32}
    op = OperatorSupport("linear", devices, dtypes, "dense")
    caps = BackendCapabilities("third-party", [op])
    devices |= {"mps"}
    dtypes |= {torch.float64}
    assert (op.device_types, op.dtypes) == (frozenset({"cpu"}), frozenset({torch.float32}))
    assert caps.operators == (op,)
    assert caps.supports("linear", dtype=torch.float32, device="cpu")
    assert not caps.supports("linear", dtype=torch.float32, device="mps")
    assert not caps.supports("linear", dtype=torch.float64, device="cpu")


@pytest.mark.parametrize(
    "build,error,text",
    [
        (lambda: OperatorSupport("linear", {"cpu"}, {torch.float32}, weight_layout="unknown"), ValueError,
         "requires an explicit format"),
        (lambda: OperatorSupport("linear", {"cpu"}, {"float32"}), TypeError, "torch.dtype"),
        (lambda: OperatorSupport("", {"cpu"}, {torch.float32}), ValueError, "operation, devices and dtypes"),
        (lambda: OperatorSupport("linear", {""}, {torch.float32}), ValueError, "nonempty strings"),
        (lambda: OperatorSupport("linear", {"cpu"}, {torch.float32}, ""), ValueError, "nonempty strings"),
        (lambda: OperatorSupport("linear", {"cpu"}, {torch.float32}, materializes_weights=1), TypeError, "must be bool"),
        (lambda: BackendCapabilities("x", ["linear"]), ValueError, "typed operators"),
        (lambda: BackendCapabilities("x", [OperatorSupport("linear", {"cpu"}, {torch.float32})], reference=1),
         TypeError, "must be bool"),
    ],
)
def test_capability_records_reject_malformed_definitions(build, error, text):
    with pytest.raises(error, match=text):
        build()


def test_backend_protocol_is_abstract():
    with pytest.raises(TypeError):
        Backend()
