"""The C-ABI library on the host (no GPU): it loads, exports every function that
include/venturi_ops.h declares with the binding's signatures, reports its
identity, sizes workspaces, and rejects bad arguments before any HIP call."""

import ctypes as C
from pathlib import Path
import re

import pytest

from venturi_amd import native

HEADER = Path(__file__).resolve().parent.parent / "include" / "venturi_ops.h"


def declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(venturi_\w+)\s*\(", text))


@pytest.fixture(scope="module")
def lib():
    return native.load()


def test_every_declared_symbol_is_exported_and_bound(lib):
    names = declared()
    assert len(names) >= 25
    handle = C.CDLL(str(native.DEFAULT_LIBRARY))
    for name in names:
        assert hasattr(handle, name), name
    assert names == set(native.SIGNATURES), names ^ set(native.SIGNATURES)


def test_identity(lib):
    assert lib.venturi_blocks_abi() == 18
    assert lib.venturi_blocks_arch() == 950
    assert lib.venturi_q4_abi() == 1
    assert lib.venturi_ada_abi() == 2


def test_workspace_sizes(lib):
    # tokens * ceil(k/32) * 36 * passes (q8_dp4a.cuh:7-13); 0 on invalid input
    assert lib.venturi_q8_dp4a_bytes(2, 33, 2) == 2 * 2 * 36 * 2
    assert lib.venturi_q8_dp4a_bytes(2048, 5120, 1) == 2048 * 160 * 36
    assert lib.venturi_q8_dp4a_bytes(0, 32, 1) == 0
    assert lib.venturi_q8_dp4a_bytes(1, 32, 3) == 0
    assert "invalid A8" in lib.error()
    # MoE: 256-byte aligned sections (seg, status, pair_slot, slot_token, slot_score, h, v)
    t, k, e, h, i = 512, 8, 128, 2048, 768
    p = t * k

    def up(v):
        return (v + 255) // 256 * 256

    want = up(4 * (e + 1)) + 256 + up(4 * p) * 2 + up(2 * p) + up(2 * p * i) + up(2 * p * h)
    assert lib.venturi_moe_q4_bytes(t, k, e, h, i) == want
    assert lib.venturi_moe_q4_bytes(t, 17, e, h, i) == 0
    assert lib.venturi_moe_q4_bytes(t, k, e, 2047, i) == 0


def test_tiled_split_workspace_sizes(lib):
    # The tiled Q8 projections split K over two workgroups only where that
    # brings the grid closer to one workgroup per CU (at most 256): 8 slots of
    # 8 bytes per (token, 16-row block) then, else no workspace.
    def slots(tokens, blocks):
        return tokens * blocks * 64

    # One token: 257-384 blocks reserve slots for long rows (107 x 2 workgroups
    # where K has at least 128 chunks); fewer or more blocks stay unsplit.
    assert lib.venturi_q8_tiled_workspace_bytes(1, 5120, 0) == slots(1, 320)
    assert lib.venturi_q8_tiled_workspace_bytes(1, 4096, 0) == 0  # 256 blocks: one per workgroup
    assert lib.venturi_q8_tiled_workspace_bytes(1, 4097, 0) == slots(1, 257)
    assert lib.venturi_q8_tiled_workspace_bytes(1, 6144, 0) == slots(1, 384)
    assert lib.venturi_q8_tiled_workspace_bytes(1, 6160, 0) == 0  # 385 blocks: 129 x 2 would pass 256
    assert lib.venturi_q8_tiled_workspace_bytes(1, 7168, 0) == 0
    assert lib.venturi_q8_tiled_workspace_bytes(4, 5120, 0) == slots(4, 320)  # 107 x 2 workgroups
    assert lib.venturi_q8_tiled_workspace_bytes(4, 7168, 0) == 0  # 224 unsplit workgroups
    assert lib.venturi_q8_tiled_workspace_bytes(32, 7168, 0) == slots(32, 448)  # 112 x 2 above 16 tokens
    assert lib.venturi_q8_tiled_workspace_bytes(16, 34816, 0) == 0
    assert lib.venturi_q8_tiled_workspace_bytes(2, 16, 0) == slots(2, 1)
    # Paired planes hold 8 gate + 8 up rows per block: same block count as the plain matrix.
    assert lib.venturi_q8_tiled_workspace_bytes(8, 100, 1) == lib.venturi_q8_tiled_workspace_bytes(8, 100, 0) == slots(8, 7)
    assert lib.venturi_q8_tiled_workspace_bytes(8, 34, 0) == 0  # 3 blocks: two workgroups either way, unsplit
    assert lib.venturi_q8_tiled_workspace_bytes(8, 35, 1) == 0
    assert "even row count" in lib.error()
    assert lib.venturi_q8_tiled_workspace_bytes(33, 64, 0) == 0
    assert "1..32 tokens" in lib.error()
    # A split launch without its workspace fails on the host.
    assert lib.venturi_q8_tiled_run(16, 16, 16, 16, 4, 5120, 64, 128, 0, None, 0, None) == -1
    assert "initialised workspace" in lib.error()
    assert lib.venturi_q8_tiled_workspace_init(None, 12, None) == -1


def test_bad_arguments_fail_before_the_device(lib):
    assert lib.venturi_q8_head_run(None, None, None, None, 1, 1, 1, 128, 0, None) == -1
    assert lib.error()
    assert lib.venturi_q8_dp4a_run(None, 0, None, None, None, 1, 1, 32, 128, 1, None) == -1
    assert lib.venturi_rms_run(None, None, None, 1, 1, 0, 1e-6, None) == -1
    assert lib.venturi_q4_gemm_run(None, None, None, None, 1, 1, 1, 128, 0, None) == -1
    assert lib.venturi_moe_q4_run(*([None] * 9), 0, 1, 1, 1, 8, 8, None) == -1
    # The expert ABI returns hipErrorInvalidValue (1), as the reference returns cudaErrorInvalidValue.
    assert lib.venturi_q4_linear(None, None, None, None, 1, 1, 1, 128, None) == 1
    assert lib.venturi_q4_decode(None, None, None, 1, 1, 100, None) == 1
    # The plugin ABI keeps its own error text.
    assert lib.venturi_q4_prepare(1, 1, 1, 5, 0) == -1
    assert b"invalid Q4" in lib.venturi_ada_error()
    assert lib.venturi_row_dequant_rows(None, None, None, None, 0, 1, 1, 128, 5, None) == -1


def test_fused_entry_points_reject_bad_arguments_on_the_host(lib):
    # venturi_q8_fused_run admission (q8_fused.cuh:188-199): count 2 or 3, a
    # workspace of the A8 size, 16-byte alignment, padded == ceil(k/128)*128.
    assert lib.venturi_q8_fused_run(None, 0, None, 2, 1, 64, 128, 1, None) == -1
    assert "invalid fused DP4A" in lib.error()
    assert lib.venturi_q8_fused_run(16, 1 << 20, 16, 1, 1, 64, 128, 1, None) == -1
    assert lib.venturi_q8_fused_run(16, 1 << 20, 16, 4, 1, 64, 128, 1, None) == -1
    assert lib.venturi_q8_fused_run(16, 1 << 20, 16, 2, 1, 64, 256, 1, None) == -1
    assert lib.venturi_swiglu_q8_quantize(None, None, None, 0, 1, 64, 256, None, None) == -1
    assert "invalid fused SwiGLU" in lib.error()


def test_fused_plan_requires_two_or_three_matrices():
    from venturi_amd.q8_fused import prepare_q8_fused

    for values in ([], [object()], [object()] * 4):
        with pytest.raises(ValueError, match="two or three"):
            prepare_q8_fused(values, tokens=1, residual_compensation=True)
