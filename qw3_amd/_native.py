"""ctypes bindings of the in-tree native libraries.

libds3_hip.so implements the C ABI declared in include/ds3_hip.h; this module
declares argument/return types for every entry point and loads the library
from qw3_amd/lib/.  Loading fails loudly: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_DIR = Path(__file__).resolve().parent / "lib"
HEADER = Path(__file__).resolve().parent.parent / "include" / "ds3_hip.h"

P = C.c_void_p          # ds3_hip_buffer_t *
U32, U64, I32, I64 = C.c_uint32, C.c_uint64, C.c_int32, C.c_int64
SZ, F, D, B, CP = C.c_size_t, C.c_float, C.c_double, C.c_bool, C.c_char_p
IP, FP = C.POINTER(C.c_int32), C.POINTER(C.c_float)

# name -> (restype, argtypes); the order follows include/ds3_hip.h
SIGNATURES: dict[str, tuple] = {
    "ds3_hip_init": (C.c_int, []),
    "ds3_hip_shutdown": (None, []),
    "ds3_hip_buffer_alloc": (P, [SZ]),
    "ds3_hip_buffer_free": (None, [P]),
    "ds3_hip_buffer_from_mmap": (P, [P, SZ]),
    "ds3_hip_buffer_view": (P, [P, SZ, SZ]),
    "ds3_hip_buffer_write": (C.c_int, [P, SZ, P, SZ]),
    "ds3_hip_buffer_read": (C.c_int, [P, SZ, P, SZ]),
    "ds3_hip_vec_matmul_f32": (C.c_int, [P, P, P, U32, U32, U64]),
    "ds3_hip_vec_matmul_quantized": (C.c_int, [P, P, P, U32, U32, U64, I32]),
    "ds3_hip_vec_matmul_f32_simd": (C.c_int, [P, P, P, U32, U32, U64]),
    "ds3_hip_vec_matmul_q8_0_simd": (C.c_int, [P, P, P, U32, U32, U64]),
    "ds3_hip_vec_matmul_q4k_simd": (C.c_int, [P, P, P, U32, U32, U64]),
    "ds3_hip_vec_matmul_q6k_simd": (C.c_int, [P, P, P, U32, U32, U64]),
    "ds3_hip_vec_matmul_q4k_half": (C.c_int, [P, P, P, U32, U32, U64]),
    "ds3_hip_matmul_quantized_batch": (C.c_int, [P, P, P, U32, U32, U32, U64, U64, I32]),
    "ds3_hip_buffer_copy_f32": (C.c_int, [P, P, SZ]),
    "ds3_hip_buffer_zero_f32": (C.c_int, [P, SZ]),
    "ds3_hip_vec_add_inplace": (C.c_int, [P, P, U32]),
    "ds3_hip_vec_add": (C.c_int, [P, P, P, U32]),
    "ds3_hip_gather_rows_f32": (C.c_int, [P, P, P, U32, U32, U32]),
    "ds3_hip_scatter_add_weighted_f32": (C.c_int, [P, P, P, P, U32, U32, U32]),
    "ds3_hip_silu_mul_f32": (C.c_int, [P, P, P, U32]),
    "ds3_hip_rms_norm": (C.c_int, [P, P, P, U32, U32, F]),
    "ds3_hip_moe_ffn": (C.c_int, [P, P, P, P, P, I32, I32, I32, U64, U64, U64,
                                  P, P, P, I32, I32, I32, U64, U64, U64,
                                  P, P, P, P, P, P, U32, U32, U32, U32, U32, U64, I32, B]),
    "ds3_hip_moe_ffn_router": (C.c_int, [P, P, P, U32, U32, U64, I32]),
    "ds3_hip_moe_ffn_experts": (C.c_int, [P, P, P, P, I32, I32, I32, U64, U64, U64,
                                          P, P, P, I32, I32, I32, U64, U64, U64,
                                          P, P, P, P, U32, U32, U32, U32, IP, FP]),
    "ds3_hip_moe_router_topk_batch": (C.c_int, [P, P, P, U32, U32, U32, B]),
    "ds3_hip_moe_router_topk_batch_tokens": (C.c_int, [P, P, P, U32, U32, U32, U32, B]),
    "ds3_hip_begin_batch": (C.c_int, []),
    "ds3_hip_end_batch": (None, []),
    "ds3_hip_debug_simulate_capture": (C.c_int, [C.c_int]),
    "ds3_hip_graph_begin": (C.c_int, []),
    "ds3_hip_graph_end": (C.c_int, [C.POINTER(C.c_void_p)]),
    "ds3_hip_graph_launch": (C.c_int, [P]),
    "ds3_hip_graph_destroy": (None, [P]),
    "ds3_hip_synchronize": (None, []),
    "ds3_hip_profile_reset": (None, []),
    "ds3_hip_profile_print": (None, [CP]),
    "ds3_hip_moe_ffn_batch": (C.c_int, [P, P, P, P, P, I32, I32, I32, U64, U64, U64, P,
                                        P, P, P, P, P, U32, U32, U32, U32, U32, U64, I32, B]),
    "ds3_hip_moe_ffn_batch_noalloc": (C.c_int, [P, P, P, P, P, I32, I32, I32, U64, U64, U64, P,
                                                P, P, P, P, P, U32, U32, U32, U32, U32, U64, I32, B]),
    "ds3_hip_noalloc_scratch_bytes": (SZ, []),
    "ds3_hip_moe_block": (C.c_int, [P, P, F, P, P, P, P, I32, I32, I32, U64, U64, U64, P,
                                    P, P, P, P, U32, U32, U32, U32, U32, U64, I32, B]),
    "ds3_hip_moe_route": (C.c_int, [P, P, P, P, P, U32, U32, U32, U32, U64, I32, B]),
    "ds3_hip_moe_bucket": (C.c_int, [P, P, U32, U32, U32, P, P, P, P, P]),
    "ds3_hip_dequantize": (C.c_int, [P, U64, I32, U64, P]),
    "ds3_hip_set_router_mode": (C.c_int, [C.c_int]),
    "ds3_hip_router_stats": (C.c_int, [C.POINTER(U64), C.POINTER(U64), C.c_int]),
    "ds3_hip_debug_grouped_lists": (C.c_int, [P, P, P, P, P, P, P, P, P]),
    "ds3_hip_debug_grouped_descs": (C.c_int, [P, P]),
    "ds3_hip_set_dense_mfma_min_rows": (C.c_int, [C.c_int]),
    "ds3_hip_set_prefill_min_tokens": (C.c_int, [C.c_int]),
    "ds3_hip_kernel_timing": (None, [C.c_int]),
    "ds3_hip_kernel_timing_reset": (None, []),
    "ds3_hip_kernel_timing_only": (None, [C.c_char_p]),
    "ds3_hip_kernel_stats": (C.c_int, [C.c_int, C.c_char_p, SZ, C.POINTER(I64), C.POINTER(D)]),
    "ds3_hip_hold_stream": (C.c_int, [D]),
    "ds3_hip_timer_start": (C.c_int, []),
    "ds3_hip_timer_stop_ms": (D, []),
    "ds3_hip_device_info": (C.c_int, [C.c_char_p, SZ, C.POINTER(C.c_int), C.POINTER(U64)]),
}

GEN_SIGNATURES: dict[str, tuple] = {
    "ds3gen_fill": (None, [C.c_int, U64, U64, U64, I64, D, D, P]),
    "ds3gen_fp32_to_fp16": (C.c_uint16, [F]),
    "ds3gen_quantize": (I64, [C.c_int, P, I64, P]),
    "ds3gen_row_bytes": (I64, [C.c_int, I64]),
    "ds3gen_matrix": (C.c_int, [C.c_int, C.c_int, U64, U64, I64, I64, D, D, P, C.c_int]),
}

_hip = None
_gen = None


def _bind(lib: C.CDLL, table: dict[str, tuple]) -> C.CDLL:
    for name, (res, args) in table.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def hip() -> C.CDLL:
    """The HIP backend (libds3_hip.so).  Raises if it was not built."""
    global _hip
    if _hip is None:
        # DS3_HIP_LIB selects another build of the same library (tuning runs)
        path = Path(os.environ.get("DS3_HIP_LIB", LIB_DIR / "libds3_hip.so"))
        if not path.exists():
            raise RuntimeError(f"{path} is missing: run python -c 'import __graft_entry__ as g; g.build()' "
                               "(there is no CPU fallback)")
        _hip = _bind(C.CDLL(str(path)), SIGNATURES)
    return _hip


def gen() -> C.CDLL:
    """The synthetic-workload generator (libds3gen.so)."""
    global _gen
    if _gen is None:
        path = LIB_DIR / "libds3gen.so"
        if not path.exists():
            raise RuntimeError(f"{path} is missing: build the package first")
        _gen = _bind(C.CDLL(str(path)), GEN_SIGNATURES)
    return _gen


def header_functions() -> list[str]:
    """Function names declared in include/ds3_hip.h."""
    import re
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ds3_hip_\w+)\s*\(", text)))
