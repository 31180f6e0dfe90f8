"""Loads libmatricxon_amd.so (built in-tree by `python -m matricxon_amd.build`) through ctypes.

torch is imported first on purpose: the library links `libamdhip64.so.7`, and torch has then
already mapped its own HIP runtime under that soname, so both share one HIP runtime (one set of
devices, streams and allocations). There is no fallback: a missing library raises.
"""

import ctypes
from pathlib import Path

import torch  # noqa: F401  (must load torch's HIP runtime before the library)

LIB_PATH = Path(__file__).resolve().parent / "libmatricxon_amd.so"

# Exported symbols, as declared in include/matricxon_amd.h.
EXPORTS = (
    "mxa_build_info",
    "mxa_supports",
    "mxa_supports_dequant_rows",
    "mxa_set_fused_max_tokens",
    "mxa_fused_max_tokens",
    "mxa_row_bytes",
    "mxa_workspace_bytes",
    "mxa_gemm",
    "mxa_gemm_static",
    "mxa_gemv_f32",
    "mxa_gemm_q8k",
    "mxa_gemm_moe",
    "mxa_gemm_moe_bf16",
    "mxa_gemm_moe_pairs",
    "mxa_gemm_moe_pairs_bf16",
    "mxa_moe_route",
    "mxa_moe_combine",
    "mxa_gemm_multi",
    "mxa_gemm_multi_q8k",
    "mxa_quantize_q8_k",
    "mxa_rms_norm_q8_k",
    "mxa_silu_mul_q8_k",
    "mxa_dequantize",
    "mxa_dequant_rows",
    "mxa_gather_rows",
    "mxa_stream_read",
    "mxa_last_error",
    "mxa_workspace_bytes_bf16",
    "mxa_gemm_bf16",
    "mxa_gemm_multi_bf16",
    "mxa_gemm_q8k_bf16",
    "mxa_gemm_multi_q8k_bf16",
    "mxa_quantize_q8_k_bf16",
    "mxa_rms_norm_q8_k_bf16",
    "mxa_silu_mul_q8_k_bf16",
)

_vp = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t
_ll = ctypes.c_longlong

_lib: ctypes.CDLL | None = None


class LibraryMissingError(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise LibraryMissingError(
            f"{LIB_PATH} is not built: run `python -m matricxon_amd.build` (hipcc, gfx950)"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    lib.mxa_build_info.argtypes = []
    lib.mxa_build_info.restype = ctypes.c_char_p
    lib.mxa_supports.argtypes = [_i, _i]
    lib.mxa_supports.restype = _i
    lib.mxa_supports_dequant_rows.argtypes = [_i, _i]
    lib.mxa_supports_dequant_rows.restype = _i
    lib.mxa_set_fused_max_tokens.argtypes = [_i]
    lib.mxa_set_fused_max_tokens.restype = None
    lib.mxa_fused_max_tokens.argtypes = []
    lib.mxa_fused_max_tokens.restype = _i
    lib.mxa_row_bytes.argtypes = [_i, _i]
    lib.mxa_row_bytes.restype = _sz
    lib.mxa_workspace_bytes.argtypes = [_i, _i, _i]
    lib.mxa_workspace_bytes.restype = _sz
    lib.mxa_gemm.argtypes = [_i, _vp, _vp, _vp, _i, _i, _i, _vp, _sz, _vp]
    lib.mxa_gemm.restype = _i
    lib.mxa_gemm_static.argtypes = [_i, _vp, _vp, _vp, _i, _i, _i, _vp]
    lib.mxa_gemm_static.restype = _i
    lib.mxa_gemv_f32.argtypes = [_i, _vp, _vp, _vp, _i, _i, _i, _vp]
    lib.mxa_gemv_f32.restype = _i
    lib.mxa_gemm_q8k.argtypes = [_i, _vp, _vp, _vp, _i, _i, _i, _vp, _sz, _vp]
    lib.mxa_gemm_q8k.restype = _i
    lib.mxa_gemm_moe.argtypes = [_i, _vp, _ll, _i, _vp, _vp, _i, _i, _vp, _i, _i, _vp, _sz, _vp]
    lib.mxa_gemm_moe.restype = _i
    lib.mxa_gemm_moe_bf16.argtypes = [_i, _vp, _ll, _i, _vp, _vp, _i, _i, _vp, _i, _i, _vp, _sz, _vp]
    lib.mxa_gemm_moe_bf16.restype = _i
    lib.mxa_gemm_moe_pairs.argtypes = [_i, _vp, _ll, _i, _vp, _i, _vp, _i, _vp, _i, _i, _vp, _sz, _vp]
    lib.mxa_gemm_moe_pairs.restype = _i
    lib.mxa_gemm_moe_pairs_bf16.argtypes = [_i, _vp, _ll, _i, _vp, _i, _vp, _i, _vp, _i, _i, _vp, _sz, _vp]
    lib.mxa_gemm_moe_pairs_bf16.restype = _i
    lib.mxa_moe_route.argtypes = [_vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp]
    lib.mxa_moe_route.restype = _i
    lib.mxa_moe_combine.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp]
    lib.mxa_moe_combine.restype = _i
    lib.mxa_gemm_multi.argtypes = [_i, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp, _sz, _vp]
    lib.mxa_gemm_multi.restype = _i
    lib.mxa_gemm_multi_q8k.argtypes = [_i, _vp, _vp, _vp, _vp, _i, _i, _vp, _sz, _vp]
    lib.mxa_gemm_multi_q8k.restype = _i
    lib.mxa_quantize_q8_k.argtypes = [_vp, _i, _i, _vp, _sz, _vp]
    lib.mxa_quantize_q8_k.restype = _i
    lib.mxa_rms_norm_q8_k.argtypes = [_vp, _vp, ctypes.c_float, _i, _i, _vp, _vp, _sz, _vp]
    lib.mxa_rms_norm_q8_k.restype = _i
    lib.mxa_workspace_bytes_bf16.argtypes = [_i, _i, _i]
    lib.mxa_workspace_bytes_bf16.restype = _sz
    lib.mxa_gemm_bf16.argtypes = [_i, _vp, _vp, _vp, _i, _i, _i, _vp, _sz, _vp]
    lib.mxa_gemm_bf16.restype = _i
    lib.mxa_gemm_multi_bf16.argtypes = [_i, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp, _sz, _vp]
    lib.mxa_gemm_multi_bf16.restype = _i
    lib.mxa_gemm_q8k_bf16.argtypes = [_i, _vp, _vp, _i, _i, _i, _vp, _sz, _vp]
    lib.mxa_gemm_q8k_bf16.restype = _i
    lib.mxa_gemm_multi_q8k_bf16.argtypes = [_i, _vp, _vp, _vp, _vp, _i, _i, _vp, _sz, _vp]
    lib.mxa_gemm_multi_q8k_bf16.restype = _i
    lib.mxa_quantize_q8_k_bf16.argtypes = [_vp, _i, _i, _vp, _sz, _vp]
    lib.mxa_quantize_q8_k_bf16.restype = _i
    lib.mxa_rms_norm_q8_k_bf16.argtypes = [_vp, _vp, ctypes.c_float, _i, _i, _vp, _vp, _sz, _vp]
    lib.mxa_rms_norm_q8_k_bf16.restype = _i
    lib.mxa_silu_mul_q8_k_bf16.argtypes = [_vp, _vp, _ll, _i, _i, _vp, _vp, _sz, _vp]
    lib.mxa_silu_mul_q8_k_bf16.restype = _i
    lib.mxa_silu_mul_q8_k.argtypes = [_vp, _vp, _ll, _i, _i, _vp, _vp, _sz, _vp]
    lib.mxa_silu_mul_q8_k.restype = _i
    lib.mxa_dequantize.argtypes = [_i, _vp, _ll, _vp, _vp]
    lib.mxa_dequantize.restype = _i
    lib.mxa_dequant_rows.argtypes = [_i, _vp, _ll, _vp, _i, _i, _vp, _vp]
    lib.mxa_dequant_rows.restype = _i
    lib.mxa_gather_rows.argtypes = [_vp, _ll, _ll, _vp, _i, _vp, _vp]
    lib.mxa_gather_rows.restype = _i
    lib.mxa_stream_read.argtypes = [_vp, _ll, _vp, _vp]
    lib.mxa_stream_read.restype = _i
    lib.mxa_last_error.argtypes = []
    lib.mxa_last_error.restype = ctypes.c_char_p
    _lib = lib
    return lib
