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
    if path == "chunked-dense":
        # fp16 ChunkedDense plans from 1024 tokens: the dense route's fixed buffer
        # (hipBLASLt's 32 MiB and 192 MiB of fp16 shadow); below that, none.
        want = (32 + 192) * 2**20
        assert plan.workspace_bytes(tokens=1023, k=5120) == 0
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


def test_dense_workspace_policy():
    # venturi_row_dense_workspace_bytes (host only): hipBLASLt's 32 MiB plus the
    # fp16 shadow of one chunk; shadows up to 192 MiB decode whole, larger ones
    # in chunks of whole 1024-row blocks within 80 MiB (at least one block).
    from venturi_amd import native

    lib = native.load()
    blas = 32 * 2**20
    assert lib.venturi_row_dense_workspace_bytes(2048, 5120, 17408) == blas + 2 * 5120 * 17408  # 170 MiB: whole
    assert lib.venturi_row_dense_workspace_bytes(2048, 34816, 5120) == blas + 2 * 8192 * 5120  # 4 + a 2048-row tail
    assert lib.venturi_row_dense_workspace_bytes(1, 248320, 5120) == blas + 2 * 8192 * 5120
    assert lib.venturi_row_dense_workspace_bytes(4096, 65536, 16384) == blas + 2 * 2048 * 16384
    assert lib.venturi_row_dense_workspace_bytes(8, 16384, 65536) == blas + 2 * 1024 * 65536  # one block at least
    assert lib.venturi_row_dense_workspace_bytes(0, 8, 8) == 0
    assert lib.venturi_row_dense_workspace_bytes(4, 8, 12) == 0 and "k % 8" in lib.error()
    assert lib.venturi_row_dense_workspace_bytes(4, 12, 8) == 0


def test_dense_bridge_create_and_destroy():
    # venturi_dense_create (blocks.cu:674-689): a plan for dtype 0/1/2, NULL with
    # the reference's message for another; destroy accepts NULL.
    from venturi_amd import native

    lib = native.load()
    for dtype in (0, 1, 2):
        plan = lib.venturi_dense_create(dtype)
        assert plan
        lib.venturi_dense_destroy(plan)
    assert not lib.venturi_dense_create(3)
    assert "unsupported scalar type" in lib.error()
    lib.venturi_dense_destroy(None)
