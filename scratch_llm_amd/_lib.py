"""ctypes binding of libsqx_hip.so (the C ABI declared in include/sqx.h).

The library is loaded after torch so that the process maps one HIP runtime (torch's); every call
passes device pointers from torch tensors and torch's current stream. Nothing here falls back to
another implementation: a missing library, a CPU tensor or a non-zero status raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libsqx_hip.so"

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2
DTYPE_F64 = 3  # sqx_nvfp4_ceil_quantize only
FP4_MX = 0
FP4_NV = 1
FP4_SCALE_MX_F32 = 0
FP4_SCALE_MX_E8M0 = 1
FP4_SCALE_NV_F32 = 2
FP4_SCALE_NV_E4M3 = 3

_TORCH_TO_SQX = {torch.float32: DTYPE_F32, torch.bfloat16: DTYPE_BF16, torch.float16: DTYPE_F16}

_c_i = ctypes.c_int
_c_i64 = ctypes.c_int64
_c_p = ctypes.c_void_p

# name -> (restype, argtypes). Kept in the order of include/sqx.h.
_SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "sqx_last_error": (ctypes.c_char_p, []),
    "sqx_abi_version": (_c_i, []),
    "sqx_int4_quantize_sym": (_c_i, [_c_p, _c_i, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p]),
    "sqx_int4_pack": (_c_i, [_c_p, _c_i64, _c_p, _c_p]),
    "sqx_int4_unpack": (_c_i, [_c_p, _c_i64, _c_p, _c_p]),
    "sqx_int4_dequantize": (_c_i, [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p]),
    "sqx_int4_tiled_weight_bytes": (_c_i64, [_c_i64, _c_i64]),
    "sqx_int4_tiled_param_count": (_c_i64, [_c_i64, _c_i64, _c_i64]),
    "sqx_int4_tile": (_c_i, [_c_p, _c_i, _c_p, _c_p, _c_i, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p]),
    "sqx_int4_tile_packed": (_c_i, [_c_p, _c_p, _c_i, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p]),
    "sqx_int4_untile": (_c_i, [_c_p, _c_p, _c_p, _c_i, _c_i, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p]),
    "sqx_int8_untile": (_c_i, [_c_p, _c_i64, _c_i64, _c_p, _c_p]),
    "sqx_fp4_untile": (_c_i, [_c_p, _c_p, _c_i, _c_i64, _c_i64, _c_p, _c_p, _c_p]),
    "sqx_mxfp4_pair_dequantize_f64": (_c_i, [_c_p, _c_p, _c_i64, _c_i64, _c_p, _c_p]),
    "sqx_int4_linear_default_kslices": (_c_i, [_c_i64, _c_i64, _c_i64]),
    "sqx_int4_linear": (
        _c_i,
        [_c_p, _c_p, _c_p, _c_i, _c_p, _c_i, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i, _c_p],
    ),
    "sqx_int4_linear_colscaled": (
        _c_i,
        [_c_p, _c_p, _c_p, _c_i, _c_p, _c_i, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i, _c_p],
    ),
    "sqx_int4_skinny_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_i]),
    "sqx_int4_skinny": (
        _c_i,
        [_c_p, _c_p, _c_p, _c_i, _c_p, _c_i, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i, _c_i, _c_i, _c_i,
         _c_p, _c_i64, _c_p],
    ),
    "sqx_int4_skinny_default_splits": (_c_i, [_c_i64, _c_i64, _c_i64]),
    "sqx_int4_skinny_partials": (_c_i, [_c_p, _c_p, _c_p, _c_i, _c_p, _c_i, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_i64,
                                        _c_p]),
    "sqx_int4_prologue_fits": (_c_i, [_c_i64, _c_i64]),
    "sqx_int4_linear_rmsnorm": (
        _c_i,
        [_c_p, _c_p, _c_p, _c_p, _c_p, ctypes.c_float, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i, _c_p],
    ),
    "sqx_int4_linear_silu": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i, _c_p]),
    "sqx_int4_linear_silu_fits": (_c_i, [_c_i64, _c_i64, _c_i64]),
    "sqx_int4_linear_residual": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64,
                                        _c_i, _c_p]),
    "sqx_int4_linear_attn_residual": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64,
                                              _c_i64, _c_i64, _c_i64, _c_i, _c_p]),
    "sqx_int4_linear_silu_residual": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64,
                                             _c_i64, _c_i, _c_p]),
    "sqx_int4_linear_rmsnorm_sumsq": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_p, ctypes.c_float, _c_p, _c_i64, _c_i64,
                                             _c_i64, _c_i64, _c_i, _c_p]),
    "sqx_int4_linear_rowscale_sumsq": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_i64, ctypes.c_float, _c_p, _c_i64, _c_i64,
                                              _c_i64, _c_i64, _c_i, _c_p]),
    "sqx_int4_linear_swiglu": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p]),
    "sqx_int4_linear_rowscale_swiglu": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_i64, ctypes.c_float, _c_p, _c_i64, _c_i64,
                                              _c_i64, _c_i64, _c_i, _c_p]),
    "sqx_int4_linear_rope_kv": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_i64, ctypes.c_float, _c_p, _c_p, _c_p, _c_i64, _c_i64,
                                       _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i, _c_p]),
    "sqx_int4_rows_fits": (_c_i, [_c_i64, _c_i64, _c_i64, _c_i]),
    "sqx_e2m1_round": (_c_i, [_c_p, _c_i, _c_i64, _c_p, _c_p]),
    "sqx_e2m1_decode": (_c_i, [_c_p, _c_i64, _c_p, _c_p]),
    "sqx_fp4_pack": (_c_i, [_c_p, _c_i64, _c_p, _c_p]),
    "sqx_fp4_unpack": (_c_i, [_c_p, _c_i64, _c_p, _c_p]),
    "sqx_quantize_e4m3": (_c_i, [_c_p, _c_i64, _c_p, _c_p]),
    "sqx_quantize_e8m0": (_c_i, [_c_p, _c_i64, _c_p, _c_p]),
    "sqx_mxfp4_quantize": (_c_i, [_c_p, _c_i, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p]),
    "sqx_mxfp4_fake_quant_rows": (_c_i, [_c_p, _c_i, _c_i64, _c_i64, _c_p, _c_p]),
    "sqx_mxfp4_dequantize": (_c_i, [_c_p, _c_p, _c_i64, _c_i64, _c_p, _c_p]),
    "sqx_nvfp4_workspace_bytes": (_c_i64, []),
    "sqx_nvfp4_quantize": (_c_i, [_c_p, _c_i, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_p]),
    "sqx_nvfp4_dequantize": (_c_i, [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_p, _c_p]),
    "sqx_fp4_tiled_weight_bytes": (_c_i64, [_c_i64, _c_i64]),
    "sqx_fp4_tiled_scale_bytes": (_c_i64, [_c_i64, _c_i64, _c_i]),
    "sqx_fp4_tile": (_c_i, [_c_p, _c_i, _c_p, _c_i, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p]),
    "sqx_fp4_linear": (
        _c_i,
        [_c_p, _c_p, _c_i, _c_p, _c_p, _c_i, _c_p, _c_i, _c_p, _c_i64, _c_i64, _c_i64, _c_i, _c_p],
    ),
    "sqx_mxfp4_quantize_tiled": (_c_i, [_c_p, _c_i, _c_i64, _c_i64, _c_p, _c_p, _c_p]),
    "sqx_mxfp4_gemm": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i, _c_p, _c_i64, _c_i64, _c_i64, _c_p]),
    "sqx_mxfp4_gemm_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_i]),
    "sqx_mxfp4_gemm_ws": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i, _c_p, _c_i64, _c_i64, _c_i64, _c_i, _c_p, _c_i64,
                                 _c_p]),
    "sqx_gemm_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64]),
    "sqx_int4_gemm": (
        _c_i,
        [_c_p, _c_p, _c_p, _c_i, _c_p, _c_i, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_p],
    ),
    "sqx_int4_linear_f32_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64]),
    "sqx_int4_linear_f32": (
        _c_i,
        [_c_p, _c_p, _c_p, _c_i, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_p],
    ),
    "sqx_fp4_gemm": (
        _c_i,
        [_c_p, _c_p, _c_i, _c_p, _c_p, _c_i, _c_p, _c_i, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_p],
    ),
    "sqx_nvfp4_ceil_quantize": (_c_i, [_c_p, _c_i, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p]),
    "sqx_nvfp4_ceil_dequantize": (_c_i, [_c_p, _c_p, _c_i64, _c_i64, _c_p, _c_i, _c_p]),
    "sqx_ue4m3_ceil": (_c_i, [_c_p, _c_i64, ctypes.c_double, _c_p, _c_p, _c_p, _c_p]),
    "sqx_e2m1_round_rne": (_c_i, [_c_p, _c_i64, _c_p, _c_p, _c_p]),
    "sqx_split_bf16": (_c_i, [_c_p, _c_i64, _c_p, _c_p, _c_p]),
    "sqx_sum_halves": (_c_i, [_c_p, _c_i64, _c_p, _c_p]),
    "sqx_int8_workspace_bytes": (_c_i64, []),
    "sqx_int8_quantize_sym": (_c_i, [_c_p, _c_i, _c_i64, _c_i64, _c_i64, ctypes.c_float, _c_p, _c_p, _c_p, _c_i64, _c_p]),
    "sqx_int8_quantize_affine": (
        _c_i,
        [_c_p, _c_i, _c_i64, _c_i64, _c_i64, ctypes.c_float, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_p],
    ),
    "sqx_int8_dequantize_sym": (_c_i, [_c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i, _c_p, _c_p]),
    "sqx_int8_dequantize_affine": (_c_i, [_c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_i, _c_p, _c_p]),
    "sqx_w8a8_gemm": (_c_i, [_c_p, _c_p, _c_i, _c_p, _c_p, _c_i, _c_p, _c_i64, _c_i64, _c_i64, _c_p]),
    "sqx_int8_tiled_weight_bytes": (_c_i64, [_c_i64, _c_i64]),
    "sqx_int8_tile": (_c_i, [_c_p, _c_i64, _c_i64, _c_p, _c_p]),
    "sqx_int8_linear": (_c_i, [_c_p, _c_p, _c_p, _c_i, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i, _c_p]),
    "sqx_int4_quantize_asym": (_c_i, [_c_p, _c_i, _c_i64, _c_i64, _c_i64, _c_i, _c_p, _c_p, _c_p, _c_p]),
    "sqx_awq_quantize": (_c_i, [_c_p, _c_i, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p]),
    "sqx_awq_fake_quant": (_c_i, [_c_p, _c_i, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p]),
    "sqx_awq_dequantize": (_c_i, [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p]),
    "sqx_col_absmean": (_c_i, [_c_p, _c_i, _c_i64, _c_i64, _c_p, _c_p]),
    "sqx_awq_scale": (_c_i, [_c_p, _c_i64, ctypes.c_float, _c_p, _c_p]),
    "sqx_scale_columns": (_c_i, [_c_p, _c_i, _c_p, _c_i64, _c_i64, _c_p, _c_p]),
    "sqx_fp8_quantize_rows": (_c_i, [_c_p, _c_i, _c_i64, _c_i64, _c_p, _c_p, _c_p]),
    "sqx_fp8_dequantize_rows": (_c_i, [_c_p, _c_p, _c_i64, _c_i64, _c_p, _c_p]),
    "sqx_fp8_head_scale": (_c_i, [_c_p, _c_i, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p]),
    "sqx_fp8_quantize_heads": (_c_i, [_c_p, _c_i, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p]),
    "sqx_fp8_dequantize_heads": (_c_i, [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p]),
    "sqx_fp8_tiled_weight_bytes": (_c_i64, [_c_i64, _c_i64]),
    "sqx_fp8_tile": (_c_i, [_c_p, _c_i64, _c_i64, _c_p, _c_p]),
    "sqx_fp8_linear_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64]),
    "sqx_fp8_skinny_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_i]),
    "sqx_fp8_skinny": (_c_i, [_c_p, _c_p, _c_p, _c_i, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i, _c_i, _c_i, _c_p, _c_i64,
                              _c_p]),
    "sqx_fp8_linear": (
        _c_i,
        [_c_p, _c_p, _c_p, _c_i, _c_p, _c_i, _c_p, _c_i64, _c_i64, _c_i64, _c_i, _c_p, _c_i64, _c_p],
    ),
    "sqx_rmsnorm": (_c_i, [_c_p, _c_p, _c_p, ctypes.c_float, _c_i64, _c_i64, _c_p, _c_p, _c_p]),
    "sqx_rmsnorm_partials": (_c_i, [_c_p, _c_p, _c_i, _c_p, ctypes.c_float, _c_i64, _c_i64, _c_p, _c_p, _c_p]),
    "sqx_rope_kv": (
        _c_i,
        [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p],
    ),
    "sqx_attn_chunk": (_c_i, [_c_i64, _c_i64, _c_i64]),
    "sqx_attn_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "sqx_attn_partials_chunk": (_c_i, [_c_i64]),
    "sqx_attn_partials_combine": (_c_i, [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p]),
    "sqx_attn_partials_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64]),
    "sqx_decode_attention_partials": (
        _c_i,
        [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_i64,
         _c_p],
    ),
    "sqx_decode_attention": (
        _c_i,
        [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_p],
    ),
    "sqx_decode_attention_rope": (
        _c_i,
        [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_p],
    ),
    "sqx_decode_attention_rope_noalloc": (
        _c_i,
        [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p],
    ),
    "sqx_decode_attention_fp8kv": (
        _c_i,
        [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_p],
    ),
    "sqx_decode_attention_rope_fp8kv": (
        _c_i,
        [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p,
         _c_i64, _c_p],
    ),
    "sqx_decode_attention_rope_parts": (
        _c_i,
        [_c_p, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p,
         _c_p, _c_i64, _c_p],
    ),
    "sqx_silu_mul":(_c_i, [_c_p, _c_i64, _c_i64, _c_p, _c_p]),
    "sqx_silu_mul_pairs8": (_c_i, [_c_p, _c_i64, _c_i64, _c_p, _c_p]),
    "sqx_embed": (_c_i, [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_p, _c_p]),
    "sqx_argmax_workspace_bytes": (_c_i64, [_c_i64, _c_i64]),
    "sqx_argmax": (_c_i, [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_p]),
    "sqx_advance": (_c_i, [_c_p, _c_p, _c_i64, _c_p]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class SqxError(RuntimeError):
    """A libsqx_hip.so call returned a non-zero status."""


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
                )
            lib = ctypes.CDLL(os.fspath(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def exported_names() -> list[str]:
    return list(_SIGNATURES)


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().sqx_last_error().decode(errors="replace")
        if rc == -1 and "not divisible" in msg:
            raise ValueError(msg)
        raise SqxError(f"{what} failed (status {rc}): {msg}")


def sqx_dtype(dt: torch.dtype) -> int:
    try:
        return _TORCH_TO_SQX[dt]
    except KeyError:
        raise TypeError(f"dtype {dt} is not supported by the HIP kernels") from None


def gemm_workspace(m: int, rows: int, cols: int, device: torch.device) -> torch.Tensor | None:
    """fp32 split-K workspace the prefill GEMMs want for this shape (None when they do not split)."""
    nb = int(load().sqx_gemm_workspace_bytes(m, rows, cols))
    return None if nb <= 0 else torch.empty(nb // 4, dtype=torch.float32, device=device)


def ws_args(ws: torch.Tensor | None) -> tuple[int | None, int]:
    return (None, 0) if ws is None else (ws.data_ptr(), ws.numel() * 4)


def require_device(*tensors: torch.Tensor | None, fn: str) -> torch.device:
    """All tensors must live on one ROCm device; returns it. CPU tensors raise RuntimeError."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"{fn}: the MI355X kernels need device tensors, got a {t.device.type} tensor "
                "(this library has no CPU path; use the reference implementation on CPU)"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"{fn}: tensors on different devices ({dev} vs {t.device})")
    if dev is None:
        raise RuntimeError(f"{fn}: no tensor argument")
    return dev


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
