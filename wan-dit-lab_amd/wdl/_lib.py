"""Loads lib/libwdl.so (the C ABI of include/wdl.h) once through ctypes and raises on any non-zero status.

The library is the only compute path: there is no fallback. A missing library raises FileNotFoundError naming the
build command, as operators.library does for the reference's DLLs (src/wan_dit_lab/kernels/operators.py:12-16).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parents[1] / "lib" / "libwdl.so"

c_i64 = ctypes.c_int64
c_int = ctypes.c_int
c_ptr = ctypes.c_void_p
c_f32 = ctypes.c_float
c_i64p = ctypes.POINTER(ctypes.c_int64)
c_i32p = ctypes.POINTER(ctypes.c_int32)

# name -> argtypes, in the order of include/wdl.h
SIGNATURES: dict[str, list] = {
    "wdl_last_error": [],
    "wdl_abi_version": [],
    "wdl_kv_append_fp8": [c_ptr, c_int, c_i64p, c_ptr, c_int, c_i64p, c_i64, c_i64, c_i64, c_i64,
                          c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_ptr],
    "wdl_act_quant_workspace_floats": [c_i64, c_i64],
    "wdl_act_quant_w4": [c_ptr, c_i64, c_i64, c_i64, c_ptr, c_f32, c_int, c_ptr, c_i64, c_ptr, c_ptr, c_ptr, c_i64,
                         c_ptr, c_ptr, c_ptr, c_ptr, c_int, c_f32, c_ptr, c_ptr, c_ptr, c_ptr],
    "wdl_act_quant_w4_static": [c_ptr, c_i64, c_i64, c_i64, c_ptr, c_f32, c_int, c_ptr, c_i64, c_ptr, c_ptr, c_ptr,
                                c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_int, c_f32, c_ptr, c_ptr, c_ptr],
    "wdl_w4a4_weight_codes": [c_ptr, c_i64, c_i64, c_ptr, c_ptr],
    "wdl_w4a4_scale_pairs": [c_ptr, c_int, c_i64, c_ptr, c_ptr],
    "wdl_w4a4_gemm_workspace_bytes": [c_i64, c_i64, c_i64],
    "wdl_w4a4_gemm": [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_i64, c_ptr,
                      c_i64, c_int, c_ptr, c_ptr, c_ptr, c_ptr],
    "wdl_w4a4_gemm_gelu_quant_workspace_floats": [c_i64, c_i64],
    "wdl_w4a4_gemm_gelu_quant": [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_i64,
                                 c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr],
    "wdl_fp8_quantize_workspace_floats": [c_i64, c_i64],
    "wdl_fp8_quantize": [c_ptr, c_int, c_i64, c_i64, c_i64, c_i64, c_int, c_ptr, c_ptr, c_ptr, c_ptr],
    "wdl_fp8_gemm_workspace_bytes": [c_i64, c_i64, c_i64],
    "wdl_fp8_gemm": [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_int, c_ptr, c_i64, c_ptr,
                     c_ptr],
    "wdl_fp8wo_gemm": [c_ptr, c_i64, c_ptr, c_ptr, c_int, c_ptr, c_i64, c_i64, c_i64, c_ptr, c_i64, c_int, c_ptr,
                       c_ptr],
    "wdl_qk_norm_rope": [c_ptr, c_i64, c_ptr, c_i64, c_ptr, c_ptr, c_ptr, c_int, c_i64, c_i64, c_i64, c_int, c_int,
                         c_int, c_int, c_f32, c_ptr, c_ptr, c_i64, c_ptr],
    "wdl_quant_q": [c_ptr, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_ptr],
    "wdl_sage_prep_workspace_floats": [c_i64, c_int],
    "wdl_sage_prep": [c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_ptr, c_i64, c_ptr, c_i64, c_i64, c_i64, c_i64, c_int,
                      c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr],
    "wdl_sage_prep_mapped": [c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_ptr, c_ptr, c_ptr, c_i64, c_ptr, c_i64, c_i64,
                             c_i64, c_i64, c_int, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr],
    "wdl_sage_cache_stats": [c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_int, c_ptr, c_ptr, c_ptr],
    "wdl_sage_prep_cached": [c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_ptr, c_i64, c_ptr, c_i64, c_i64, c_i64, c_i64,
                             c_ptr, c_int, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr],
    "wdl_sage_prep_cached_append": [c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_ptr, c_i64, c_ptr, c_i64, c_i64, c_i64,
                                    c_i64, c_ptr, c_int, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr],
    "wdl_sage_sm89_relayout": [c_ptr, c_i64, c_ptr, c_i64, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_ptr],
    "wdl_sage_attn_workspace_bytes": [c_i64, c_i64, c_i64],
    "wdl_sage_attn": [c_ptr, c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_f32, c_ptr, c_i64,
                      c_ptr, c_ptr],
    "wdl_sage_attn_q16": [c_ptr, c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_f32, c_ptr, c_i64,
                          c_ptr, c_ptr],
    "wdl_sage_attn_q16_framed": [c_ptr, c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_f32, c_i64, c_ptr,
                                 c_i64, c_ptr, c_ptr],
    "wdl_rope3d_rotate": [c_ptr, c_int, c_i64p, c_ptr, c_int, c_i64p, c_i64, c_i64, c_i64, c_i64, c_i64, c_i32p,
                          c_i64, c_int, c_ptr, c_int, c_ptr],
    "wdl_attn_bf16_prep_elems": [c_i64, c_i64],
    "wdl_attn_bf16_prep": [c_ptr, c_i64, c_ptr, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_ptr],
    "wdl_attn_bf16": [c_ptr, c_i64, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_f32, c_ptr, c_i64, c_ptr],
}
# return types other than int: the workspace-size queries return int64_t (a c_int default would truncate them)
RESTYPES = {"wdl_last_error": ctypes.c_char_p, "wdl_sage_prep_workspace_floats": c_i64,
            "wdl_sage_attn_workspace_bytes": c_i64, "wdl_w4a4_gemm_workspace_bytes": c_i64,
            "wdl_act_quant_workspace_floats": c_i64, "wdl_fp8_quantize_workspace_floats": c_i64,
            "wdl_w4a4_gemm_gelu_quant_workspace_floats": c_i64, "wdl_attn_bf16_prep_elems": c_i64,
            "wdl_fp8_gemm_workspace_bytes": c_i64}

_LIB = None


def library() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(f"{LIB_PATH} is not built: python -m wdl.build (or __graft_entry__.build())")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, args in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = RESTYPES.get(name, c_int)
        _LIB = lib
    return _LIB


def exported_symbols() -> list[str]:
    return list(SIGNATURES)


def call(name: str, *args) -> None:
    """Calls wdl_<name>; a non-zero status raises RuntimeError with the library's message."""
    lib = library()
    status = getattr(lib, name)(*args)
    if status != 0:
        message = lib.wdl_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed ({status}): {message}")


def i64s(values) -> ctypes.Array:
    return (ctypes.c_int64 * len(values))(*[int(v) for v in values])


def i32s(values) -> ctypes.Array:
    return (ctypes.c_int32 * len(values))(*[int(v) for v in values])
