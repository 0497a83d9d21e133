"""ctypes binding of libqmm.so (the C ABI declared in include/qmm.h).

The library is built in-tree (``swarmllm_amd/libqmm.so``) by
``swarmllm_amd.build.build_library()``. Loading fails loudly when it is
missing: there is no fallback path. SWARMLLM_QMM_LIB names another build of
the same library to load instead (the host-AddressSanitizer build of
``make asan`` in csrc/).
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("SWARMLLM_QMM_LIB") or os.path.join(HERE, "libqmm.so")

QMM_OK, QMM_UNSUPPORTED, QMM_WORKSPACE_TOO_SMALL, QMM_DEVICE_ERROR, QMM_NO_TILE, QMM_NO_ROOM = range(6)
STATUS_NAMES = {0: "OK", 1: "UNSUPPORTED", 2: "WORKSPACE_TOO_SMALL", 3: "DEVICE_ERROR", 4: "NO_TILE", 5: "NO_ROOM"}
ACT_Q8K, ACT_Q8_0 = 0, 1
GLU_SILU, GLU_SWIGLU_OAI, GLU_GELU = 0, 1, 2
X_F16, X_BF16, X_F32 = 0, 1, 2


class QmmError(RuntimeError):
    def __init__(self, fn: str, status: int):
        super().__init__(f"{fn}: status {status} ({STATUS_NAMES.get(status, '?')})")
        self.status = status


_P, _I64, _I, _SZ, _U64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t, ctypes.c_uint64

# name -> (restype, argtypes); the exports of include/qmm.h
SIGNATURES = {
    "qmm_available": (_I, []),
    "qmm_act_layout": (_I, [_I, _I64]),
    "qmm_act_bytes": (_SZ, [_I, _I64, _I64]),
    "qmm_act_planes": (_I, [_I, _I64, _I64, ctypes.POINTER(_SZ), ctypes.POINTER(_SZ), ctypes.POINTER(_SZ)]),
    "qmm_quantize_act": (_I, [_P, _P, _I, _I64, _I64, _I64, _I64]),
    "qmm_matvec_max_rows": (_I, []),
    "qmm_mmq_few_rows_line": (_I, [_I, ctypes.POINTER(_I64), ctypes.POINTER(_I64)]),
    "qmm_mmq_max_rows": (_I64, []),
    "qmm_mmq_captured": (_I, []),
    "qmm_exact_forms": (_I, []),
    "qmm_set_force_dmmv": (None, [_I]),
    "qmm_force_dmmv": (_I, []),
    "qmm_matvec": (_I, [_I, _P, _P, _P, _I64, _I64, _I64, _I64, _I64]),
    "qmm_matmul": (_I, [_I, _P, _P, _P, _I64, _I64, _I64, _I64, _I64]),
    "qmm_forward": (_I, [_I, _P, _P, _I64, _P, _I64, _P, _SZ, ctypes.POINTER(_SZ), _I64, _I64, _I64, _I, _I64]),
    "qmm_forward_shared": (_I, [_I, _I, ctypes.POINTER(_P), ctypes.POINTER(_I64), ctypes.POINTER(_P),
                                ctypes.POINTER(_I64), _P, _I64, _P, _SZ, ctypes.POINTER(_SZ), _I64, _I64, _I, _I64]),
    "qmm_moe_forward": (_I, [_I, _P, _I, _P, _I64, _P, _P, _P, _I, _P, _I64, _P, _SZ, ctypes.POINTER(_SZ), _I64,
                             _I64, _I64, _I, _I64]),
    "qmm_moe_forward_prefill": (_I, [_I, _P, _I, _P, _I, _I64, _P, _P, _P, _I, _P, _I64, _P, _SZ,
                                     ctypes.POINTER(_SZ), _I64, _I64, _I64, _I, _I64]),
    "qmm_dequantize": (_I, [_I, _P, _P, _I, _I64, _I64]),
    "qmm_quantize_scratch_bytes": (_SZ, [_I, _I64]),
    "qmm_quantize_weights": (_I, [_I, _P, _P, _I64, _P, _SZ, _I64]),
    "qmm_type_bytes": (_SZ, [_I, _I64]),
    "qmm_block_size": (_I, [_I]),
    "qmm_fail_next_launch": (None, []),
    "qmm_fill_normal": (_I, [_P, _I64, _U64, ctypes.c_float, ctypes.c_float, _I64]),
    "qmm_matvec_launches": (_U64, []),
    "qmm_gemm_launches": (_U64, []),
    "qmm_moe_launches": (_U64, []),
    "qmm_moe_prefill_launches": (_U64, []),
    "qmm_last_kernel": (ctypes.c_char_p, []),
    "qmm_forward_noalloc": (_I, [_I, _P, _P, _I64, _P, _I64, _I64, _I64, _I64, _I64]),
    "qmm_forward_noalloc_max_bytes": (_SZ, []),
    "qmm_wire_bytes": (_SZ, [_I64]),
    "qmm_wire_encode": (_I, [_P, _I64, _P, _I64]),
    "qmm_wire_decode": (_I, [_P, _SZ, _I64, _P, _I64]),
    "qmm_forward_glu": (_I, [_I, _I, _P, _P, _P, _I64, _P, _I64, _P, _SZ, ctypes.POINTER(_SZ), _I64, _I64, _I64,
                             _I, _I64]),
    "qmm_glu": (_I, [_I, _P, _P, _P, _I64, _I64]),
    "qmm_gguf_open": (_I, [ctypes.c_char_p, ctypes.POINTER(_P)]),
    "qmm_gguf_close": (None, [_P]),
    "qmm_gguf_version": (_I, [_P]),
    "qmm_gguf_alignment": (ctypes.c_uint64, [_P]),
    "qmm_gguf_data_offset": (ctypes.c_uint64, [_P]),
    "qmm_gguf_tensor_count": (_I64, [_P]),
    "qmm_gguf_find_tensor": (_I64, [_P, ctypes.c_char_p]),
    "qmm_gguf_tensor_name": (ctypes.c_char_p, [_P, _I64]),
    "qmm_gguf_tensor_info": (_I, [_P, _I64, ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I64),
                                  ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    "qmm_gguf_kv_count": (_I64, [_P]),
    "qmm_gguf_find_kv": (_I64, [_P, ctypes.c_char_p]),
    "qmm_gguf_kv_key": (ctypes.c_char_p, [_P, _I64]),
    "qmm_gguf_kv_type": (_I, [_P, _I64, ctypes.POINTER(_I), ctypes.POINTER(_I64)]),
    "qmm_gguf_kv_get": (_I, [_P, _I64, _I64, ctypes.POINTER(_I64), ctypes.POINTER(ctypes.c_double),
                             ctypes.POINTER(ctypes.c_char_p)]),
    "qmm_padded_bytes": (_SZ, [_I, _I64]),
    "qmm_gguf_load": (_I, [_P, _I64, _P, _SZ, _I64]),
    "qmm_pinned_load_chunks": (_U64, []),
    "qmm_gguf_load_entries": (_I, [_P, _I64, _I64, ctypes.POINTER(_I64), _P, _SZ, _I64]),
    "qmm_load_entries": (_I, [_I, _I64, _SZ, _I64, ctypes.POINTER(_I64), ctypes.POINTER(_P), _P, _SZ, _I64]),
    "qmm_load_beside": (_I, [_I, _P, _SZ, _P, _SZ, _I64, _I64]),
    "qmm_prepare": (_I, [_I]),
    "qmm_prepared": (_I, [_I]),
    "qmm_accumulate_in_f32": (_I, [_I]),
    "qmm_gather_row_bytes": (_I, [_I, _I64, ctypes.POINTER(_SZ)]),
    "qmm_gather_rows": (_I, [_I, _P, _SZ, _I64, _I64, _P, _I64, _P, _SZ, _P, _I64]),
    "qmm_read_floor_sink_bytes": (_SZ, []),
    "qmm_read_floor": (_I, [_P, _SZ, _P, _SZ, _P, _I64]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                "(there is no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(fn: str, status: int) -> None:
    if status != QMM_OK:
        raise QmmError(fn, status)
