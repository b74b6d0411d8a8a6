"""The native plan table's admission (rowcodec::prepare, row_codec_dispatch.cuh:30-64) on the host."""

import ctypes as C

import pytest

from venturi_amd.rowcodec import VRCPlan, prepare_row_codec


@pytest.mark.parametrize(
    "bits,group,precision,dtype,impl,path,passes",
    [
        (8, 32, "wxa16", 0, "auto", "direct", 0),
        (8, 32, "wxa16", 1, "auto", "direct", 0),
        (8, 32, "wxa8", 0, "auto", "quantized", 1),
        (8, 32, "wxa8-residual", 0, "auto", "quantized", 2),
        (4, 64, "wxa16", 0, "auto", "chunked-dense", 0),
        (5, 64, "wxa16", 0, "dequant", "chunked-dense", 0),
        (6, 64, "wxa16", 0, "auto", "chunked-dense", 0),
        (4, 64, "wxa16", 0, "fused-research", "direct", 0),
    ],
)
def test_admitted_plans(bits, group, precision, dtype, impl, path, passes):
    plan = prepare_row_codec(bits, group, precision=precision, dtype=dtype, implementation=impl)
    assert plan.path == path and plan.passes == passes
    assert (plan.raw.bits, plan.raw.group, plan.raw.dtype) == (bits, group, dtype)
    want = 2048 * 160 * 36 * passes if passes else 0
    assert plan.workspace_bytes(tokens=2048, k=5120) == want


@pytest.mark.parametrize(
    "bits,group,precision,dtype,impl,reason",
    [
        (8, 32, "wxa8", 1, "auto", "fp16"),             # A8 takes fp16 only
        (8, 32, "wxa16", 0, "dequant", "Auto"),        # q8 plans: Auto only
        (8, 32, "wxa16", 2, "auto", "fp16 or bf16"),    # fp32 activations
        (4, 64, "wxa16", 1, "auto", "fp16"),            # q4-q6 take fp16 only
        (5, 64, "wxa8", 0, "auto", "A8"),               # q5 A8 is an SM70 kernel
        (5, 64, "wxa16", 0, "fused-research", "q4 only"),
        (6, 64, "wxa16", 0, "fused-research", "q4 only"),
        (7, 64, "wxa16", 0, "auto", "bits, group"),
        (4, 32, "wxa16", 0, "auto", "bits, group"),
        (8, 64, "wxa16", 0, "auto", "bits, group"),
    ],
)
def test_rejected_plans(bits, group, precision, dtype, impl, reason):
    with pytest.raises(ValueError, match=reason):
        prepare_row_codec(bits, group, precision=precision, dtype=dtype, implementation=impl)


def test_forged_plans_fail_before_the_device():
    plan = prepare_row_codec(8, 32, precision="wxa8")
    lib = plan.lib
    forged = VRCPlan(8, 32, 1, 0, 0, 0, 1)  # quantized precision with a direct path
    assert lib.venturi_rowcodec_workspace_bytes(C.byref(forged), 4, 64) == 0
    assert "does not come from prepare" in lib.error()
    assert lib.venturi_rowcodec_project(C.byref(forged), *([None] * 6), 0, 1, 1, 64, 128, 0, None) == -1
    direct = prepare_row_codec(4, 64)
    assert lib.venturi_rowcodec_project(C.byref(direct.raw), *([None] * 6), 0, 1, 1, 64, 128, 1, None) == -1
    assert "packed" in lib.error()
    assert lib.venturi_rowcodec_project(None, *([None] * 6), 0, 1, 1, 64, 128, 0, None) == -1
