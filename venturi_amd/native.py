"""ctypes binding of libventuri_ops.so, the gfx950 C-ABI library.

The library is built in-tree (``venturi_amd/_lib``) by ``__graft_entry__.build``
or ``make -C venturi_amd/csrc``. Loading fails loudly when it is missing: no
operator in this package has a CPU or PyTorch substitute.
"""

import ctypes as C
import os
from pathlib import Path
import threading

ABI_VERSION = 18
ARCH_TAG = 950

DEFAULT_LIBRARY = Path(__file__).resolve().parent / "_lib" / "libventuri_ops.so"

_P = C.c_void_p
_I = C.c_int
_U64 = C.c_uint64
_F = C.c_float

# name -> (argtypes, restype); signatures match include/venturi_ops.h.
SIGNATURES = {
    "venturi_blocks_abi": ([], _I),
    "venturi_blocks_arch": ([], _I),
    "venturi_blocks_error": ([], C.c_char_p),
    "venturi_q8_head_run": ([_P] * 4 + [_I] * 5 + [_P], _I),
    "venturi_q8_embedding_run": ([_P] * 4 + [_I] * 5 + [_P], _I),
    "venturi_q8_dp4a_bytes": ([_I] * 3, _U64),
    "venturi_q8_dp4a_quantize": ([_P, _P, _U64] + [_I] * 3 + [_P], _I),
    "venturi_q8_dp4a_run": ([_P, _U64] + [_P] * 3 + [_I] * 5 + [_P], _I),
    "venturi_q8_a8_gemm_run": ([_P, _U64] + [_P] * 3 + [_I] * 5 + [_P], _I),
    "venturi_q8_a8_tiled_run": ([_P, _U64] + [_P] * 3 + [_I] * 5 + [_P, _U64, _P], _I),
    "venturi_q8_a8_tiled_linear_run": ([_P, _P, _U64] + [_P] * 3 + [_I] * 5 + [_P, _U64, _P], _I),
    "venturi_q8_a8_tiled_workspace_bytes": ([_I] * 4, _U64),
    "venturi_q8_fused_run": ([_P, _U64, _P] + [_I] * 5 + [_P], _I),
    "venturi_swiglu_q8_quantize": ([_P] * 3 + [_U64] + [_I] * 3 + [_P, _P], _I),
    "venturi_rms_run": ([_P] * 3 + [_I] * 3 + [_F, _P], _I),
    "venturi_rms_q8_quantize": ([_P] * 3 + [_U64, _I, _I, _F, _I, _P, _P], _I),
    "venturi_rms_q8_quantize_passes": ([_P] * 3 + [_U64, _I, _I, _F, _I, _P, _P], _I),
    "venturi_q8_pack_run": ([_P] * 3 + [_I] * 4 + [_P], _I),
    "venturi_q8_gemm_run": ([_P] * 4 + [_I] * 5 + [_P], _I),
    "venturi_q8_prefill_run": ([_P] * 4 + [_I] * 5 + [_P], _I),
    "venturi_q8_tiled_workspace_bytes": ([_I] * 3, _U64),
    "venturi_q8_tiled_workspace_init": ([_P, _U64, _P], _I),
    "venturi_q8_tiled_run": ([_P] * 4 + [_I] * 5 + [_P, _U64, _P], _I),
    "venturi_q8_tiled_swiglu_run": ([_P] * 4 + [_I] * 5 + [_P, _U64, _P], _I),
    "venturi_q8_tiled_run_noalloc": ([_P] * 4 + [_I] * 5 + [_P], _I),
    "venturi_q4_pack_run": ([_P] * 3 + [_I] * 4 + [_P], _I),
    "venturi_q4_abi": ([], _I),
    "venturi_q4_decode": ([_P] * 3 + [_I] * 3 + [_P], _I),
    "venturi_q4_linear": ([_P] * 4 + [_I] * 4 + [_P], _I),
    "venturi_q4_fused_run": ([_P] * 4 + [_I] * 5 + [_P], _I),
    "venturi_row_dequant_rows": ([_P] * 4 + [_I] * 5 + [_P], _I),
    "venturi_row_dequant_indexed": ([_P] * 5 + [_I] * 4 + [_P], _I),
    "venturi_q5_abi": ([], _I),
    "venturi_q5_decode": ([_P] * 4 + [_I] * 3 + [_P], _I),
    "venturi_q5_linear": ([_P] * 5 + [_I] * 4 + [_P], _I),
    "venturi_ada_abi": ([], _I),
    "venturi_ada_error": ([], C.c_char_p),
    "venturi_q4_prepare": ([_I] * 5, _I),
    "venturi_q4_run": ([_P] * 4 + [_I] * 6 + [_P], _I),
    "venturi_q4_gemm_run": ([_P] * 4 + [_I] * 5 + [_P], _I),
    "venturi_q4_tiled_run": ([_P] * 4 + [_I] * 5 + [_P, _U64, _P], _I),
    "venturi_q4_tiled_workspace_bytes": ([_I] * 3, _U64),
    "venturi_row_tiled_run": ([_P] * 5 + [_I] * 6 + [_P, _U64, _P], _I),
    "venturi_q4_tiled_workspace_init": ([_P, _U64, _P], _I),
    "venturi_row_gemm_run": ([_P] * 5 + [_I] * 6 + [_P], _I),
    "venturi_row_dense_workspace_bytes": ([_I] * 3, _U64),
    "venturi_row_dense_run": ([_P] * 5 + [_I] * 6 + [_P, _U64, _P], _I),
    "venturi_q8_dense_workspace_bytes": ([_I] * 3, _U64),
    "venturi_dense_create": ([_I], _P),
    "venturi_dense_destroy": ([_P], None),
    "venturi_dense_run": ([_P] * 4 + [_I] * 3 + [_P, C.c_size_t, _P], _I),
    "venturi_q8_dense_run": ([_P] * 4 + [_I] * 5 + [_P, _U64, _P], _I),
    "venturi_rowcodec_prepare": ([_I] * 5 + [_P], _I),
    "venturi_rowcodec_workspace_bytes": ([_P, _I, _I], _U64),
    "venturi_rowcodec_project": ([_P] * 7 + [_U64] + [_I] * 5 + [_P], _I),
    "venturi_moe_q4_bytes": ([_I] * 5, _U64),
    "venturi_moe_q4_run": ([_P] * 9 + [_U64] + [_I] * 5 + [_P], _I),
    "venturi_silu_mul_run": ([_P] * 2 + [_I] * 3 + [_P], _I),
    "venturi_swiglu_run": ([_P] * 3 + [C.c_int64, _I, _P], _I),
    "venturi_add_run": ([_P] * 3 + [C.c_int64, _I, _P], _I),
    # Reference exports outside the quantized-linear path: present so a binding
    # of the reference's whole table loads; each call returns -1 with a message.
    "venturi_greedy_run": ([_P] * 3 + [C.c_size_t] + [_I] * 3 + [_P], _I),
    "venturi_fp32_linear_run": ([_P] * 3 + [_I] * 4 + [_P], _I),
    "venturi_rope_run": ([_P] * 4 + [_I] * 6 + [_P], _I),
    "venturi_qwen_qk_run": ([_P] * 8 + [_I] * 6 + [_F, _P], _I),
    "venturi_qwen_gate_run": ([_P] * 3 + [_I] * 4 + [_P], _I),
    "venturi_attention_run": ([_P] * 4 + [_I] * 6 + [_F, _P], _I),
    "venturi_embedding_run": ([_P] * 3 + [_I] * 4 + [_P], _I),
    "venturi_gdn_run": ([_P] * 8 + [_I] * 8 + [_F, _P], _I),
    "venturi_conv_run": ([_P] * 5 + [_I] * 5 + [_P], _I),
    "venturi_gates_run": ([_P] * 6 + [_I] * 4 + [_P], _I),
    "venturi_gated_rms_run": ([_P] * 4 + [_I] * 5 + [_F, _P], _I),
}

_lock = threading.Lock()
_loaded = {}


class NativeLibrary:
    """One loaded library with typed entry points and the error channel."""

    def __init__(self, path):
        self.path = Path(path).expanduser().resolve()
        if not self.path.is_file():
            raise FileNotFoundError(
                f"{self.path} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `make -C venturi_amd/csrc` (there is no CPU fallback)"
            )
        self.handle = C.CDLL(str(self.path))
        for name, (args, result) in SIGNATURES.items():
            try:
                function = getattr(self.handle, name)
            except AttributeError as error:
                raise RuntimeError(f"{self.path} lacks export {name}; rebuild the library") from error
            function.argtypes, function.restype = args, result
            setattr(self, name, function)
        if self.venturi_blocks_abi() != ABI_VERSION:
            raise RuntimeError("Venturi blocks ABI mismatch; rebuild explicitly")
        if self.venturi_blocks_arch() != ARCH_TAG:
            raise RuntimeError("Library is not built for gfx950")

    def error(self):
        return self.venturi_blocks_error().decode("utf-8", "replace")

    def check(self, status):
        if status < 0:
            raise RuntimeError(self.error())
        return status


def load(path=None):
    """Loads (once per path) the in-tree library or an explicit one."""
    target = Path(path or os.environ.get("VENTURI_OPS_LIBRARY") or DEFAULT_LIBRARY).expanduser().resolve()
    with _lock:
        if target not in _loaded:
            _loaded[target] = NativeLibrary(target)
        return _loaded[target]
