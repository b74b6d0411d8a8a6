"""The reference's own Python binding loads this library (CPU, no GPU).

``CudaBackend.__init__`` (/root/reference/src/venturi/ops/blocks.py:323-427)
checks the ABI number, reads the architecture tag and then binds every name of
its signature table with ``getattr``, with no fallback. The table below
restates that interface data (names, ctypes argument lists and result types,
blocks.py:336-424) so the test needs nothing from the reference at run time.
Binding it against the built library must succeed for every name, and the
names outside the quantized-linear path must answer -1 with a message instead
of touching the device.
"""

import ctypes as C

import pytest

from venturi_amd import native

P, I, F, S, I64 = C.c_void_p, C.c_int, C.c_float, C.c_size_t, C.c_int64

REFERENCE_TABLE = {
    "venturi_blocks_abi": ([], I),
    "venturi_blocks_error": ([], C.c_char_p),
    "venturi_greedy_run": ([P] * 3 + [S] + [I] * 3 + [P], I),
    "venturi_fp32_linear_run": ([P] * 3 + [I] * 4 + [P], I),
    "venturi_dense_create": ([I], P),
    "venturi_dense_destroy": ([P], None),
    "venturi_dense_run": ([P] * 4 + [I] * 3 + [P, S, P], I),
    "venturi_rms_run": ([P] * 3 + [I] * 3 + [F, P], I),
    "venturi_swiglu_run": ([P] * 3 + [I64, I, P], I),
    "venturi_rope_run": ([P] * 4 + [I] * 6 + [P], I),
    "venturi_qwen_qk_run": ([P] * 8 + [I] * 6 + [F, P], I),
    "venturi_qwen_gate_run": ([P] * 3 + [I] * 4 + [P], I),
    "venturi_attention_run": ([P] * 4 + [I] * 6 + [F, P], I),
    "venturi_q8_embedding_run": ([P] * 4 + [I] * 5 + [P], I),
    "venturi_q8_head_run": ([P] * 4 + [I] * 5 + [P], I),
    "venturi_embedding_run": ([P] * 3 + [I] * 4 + [P], I),
    "venturi_gdn_run": ([P] * 8 + [I] * 8 + [F, P], I),
    "venturi_conv_run": ([P] * 5 + [I] * 5 + [P], I),
    "venturi_gates_run": ([P] * 6 + [I] * 4 + [P], I),
    "venturi_gated_rms_run": ([P] * 4 + [I] * 5 + [F, P], I),
    "venturi_add_run": ([P] * 3 + [I64, I, P], I),
}

OUTSIDE_PATH = ["venturi_greedy_run", "venturi_fp32_linear_run", "venturi_rope_run", "venturi_qwen_qk_run",
                "venturi_qwen_gate_run", "venturi_attention_run", "venturi_embedding_run", "venturi_gdn_run",
                "venturi_conv_run", "venturi_gates_run", "venturi_gated_rms_run"]


@pytest.fixture(scope="module")
def handle():
    native.load()  # builds nothing; fails loudly if the library is missing
    return C.CDLL(str(native.DEFAULT_LIBRARY))


def test_reference_table_binds(handle):
    handle.venturi_blocks_abi.restype = I
    handle.venturi_blocks_arch.restype = I
    assert handle.venturi_blocks_abi() == 18
    # The reference accepts 70 / 89; the gfx950 backend's one gate edit accepts 950.
    assert handle.venturi_blocks_arch() == 950
    for name, (args, result) in REFERENCE_TABLE.items():
        function = getattr(handle, name)  # AttributeError here is what the reference backend would raise
        function.argtypes, function.restype = args, result


def test_reference_table_agrees_with_this_binding():
    for name, (args, result) in REFERENCE_TABLE.items():
        ours_args, ours_result = native.SIGNATURES[name]
        assert [C.sizeof(a) for a in args] == [C.sizeof(a) for a in ours_args], name
        assert (result is None) == (ours_result is None), name


@pytest.mark.parametrize("name", OUTSIDE_PATH)
def test_names_outside_the_path_fail_with_a_message(handle, name):
    args, result = REFERENCE_TABLE[name]
    function = getattr(handle, name)
    function.argtypes, function.restype = args, result
    handle.venturi_blocks_error.restype = C.c_char_p
    zeros = [0.0 if a is F else None if a is P else 0 for a in args]
    assert function(*zeros) == -1
    message = handle.venturi_blocks_error().decode()
    assert name in message and "not built for gfx950" in message
