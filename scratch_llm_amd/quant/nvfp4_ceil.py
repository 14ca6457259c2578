"""The second NVFP4 convention on MI355X: the operands of scratch_llm's b_r6 GEMM rung.

The API of ``src/scratch_llm/kernels/gemm/cuda/b_r6.py`` (``NVFP4Operand``, ``quantize_nvfp4``,
``dequantize_nvfp4``, ``b_r6_gemm_packed``, ``b_r6_gemm``, ``reference_gemm``) and the scalar rules of
``src/scratch_llm/kernels/gemm/nvfp4_layout.py:341-416`` (``ue4m3_ceil_code``, ``scale_for_amax``,
``e2m1_round_code``), computed by libsqx_hip.so on ROCm device tensors:

* per block of ``SF_VEC_SIZE = 16`` along k, in float64: ``scale = ceil_ue4m3(amax / 6)`` (no global
  scale), ``code = round_to_nearest_even_e2m1(x / scale)``, zero always as code 0, the lower k in
  the low nibble. NaN / Inf inputs and blocks with ``amax / 6 > 448`` raise ``ValueError``, as the
  reference does (the kernel flags them; the call synchronises to read the flag).
* The scale bytes are a row-major ``[rows, k/16]`` array of UE4M3 codes. The reference stores them
  in the CUTLASS tile swizzle its sm120 kernel reads; this build's kernels read their own tiled
  layout, so the swizzle is not reproduced (``NVFP4Operand.scales`` differs in layout, not in
  values).
* ``b_r6_gemm_packed`` multiplies two operands with fp32 accumulation and an fp32 result, as the
  reference's kernel: every NVFP4 value (a 2-bit-significand E2M1 times a 4-bit-significand scale) is
  exact in bf16, so A is decoded to bf16 and B runs as an NVFP4 weight with its E4M3 scale bytes and
  a global scale of 1 through the library's FP4 linear kernels. The products are exact; only the
  fp32 summation order differs from ``dequantize(A) @ dequantize(B).T``.

The scalar helpers take device tensors (float64 after conversion) and return code tensors; the
reference's take Python floats.
"""

from __future__ import annotations

import torch
from torch import Tensor

from scratch_llm_amd import _lib
from scratch_llm_amd.quant import _device
from scratch_llm_amd.quant.nvfp4_mxfp4 import FP4Tiled, fp4_linear_tiled

__all__ = [
    "E2M1_MAGNITUDES",
    "E2M1_MAX",
    "E2M1_UNIT_ROUNDOFF",
    "NVFP4Operand",
    "SF_VEC_SIZE",
    "UE4M3_CEIL_RELATIVE",
    "UE4M3_MAX",
    "UE4M3_MIN_NORMAL",
    "UE4M3_MIN_POSITIVE",
    "b_r6_gemm",
    "b_r6_gemm_packed",
    "dequantize_nvfp4",
    "e2m1_round_code",
    "quantize_nvfp4",
    "reference_gemm",
    "scale_for_amax",
    "ue4m3_ceil_code",
]

SF_VEC_SIZE = 16  # nvfp4_layout.py:149
E2M1_MAGNITUDES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)
E2M1_MAX = 6.0
E2M1_UNIT_ROUNDOFF = 0.25
UE4M3_CEIL_RELATIVE = 0.125
UE4M3_MAX = 448.0
UE4M3_MIN_POSITIVE = 2.0**-9
UE4M3_MIN_NORMAL = 2.0**-6

_NON_FINITE, _RANGE = 1, 2


class NVFP4Operand:
    """A quantized ``[rows, k]`` operand (b_r6.py NVFP4Operand): ``packed`` uint8 ``[rows, k/2]``
    (two E2M1 codes per byte, lower k in the low nibble) and ``scales`` uint8 ``[rows, k/16]``
    (UE4M3 codes, row-major)."""

    __slots__ = ("k", "packed", "rows", "scales")

    def __init__(self, packed: Tensor, scales: Tensor, rows: int, k: int) -> None:
        if k % SF_VEC_SIZE:
            raise ValueError(f"k={k} is not a multiple of SF_VEC_SIZE={SF_VEC_SIZE}")
        if packed.dtype != torch.uint8 or tuple(packed.shape) != (rows, k // 2):
            raise ValueError(f"packed must be uint8 [{rows}, {k // 2}], expected from rows={rows}, k={k}; "
                             f"got {packed.dtype} {tuple(packed.shape)}")
        if scales.dtype != torch.uint8 or tuple(scales.shape) != (rows, k // SF_VEC_SIZE):
            raise ValueError(f"scales must be uint8 [{rows}, {k // SF_VEC_SIZE}] (row-major UE4M3 codes), "
                             f"got {scales.dtype} {tuple(scales.shape)}")
        self.packed, self.scales, self.rows, self.k = packed, scales, rows, k


def _stream(t: Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _raise_on(status: Tensor, what: str) -> None:
    st = int(status.item())
    if st & _NON_FINITE:
        raise ValueError(f"{what}: operand contains NaN or Inf, and E2M1 encodes neither (NanInfEncoding::NONE)")
    if st & _RANGE:
        raise ValueError(f"{what}: a block's amax/{E2M1_MAX:g} exceeds UE4M3's maximum {UE4M3_MAX:g}; the scale is "
                         "unrepresentable — rescale the operand")


def quantize_nvfp4(x: Tensor) -> NVFP4Operand:
    """``[rows, k]`` real -> NVFP4 with ceil-rounded UE4M3 block scales (b_r6.py:155-225). Raises on a
    non-2-D operand, ``k % 16 != 0``, NaN / Inf, or an unrepresentable block."""
    if x.ndim != 2:
        raise ValueError(f"quantize_nvfp4 expects a 2-D operand, got {x.ndim}-D")
    rows, k = int(x.shape[0]), int(x.shape[1])
    if k % SF_VEC_SIZE:
        raise ValueError(f"quantize_nvfp4: K={k} is not a multiple of SF_VEC_SIZE={SF_VEC_SIZE}; a partial "
                         "scale block has no encoding")
    dev = _lib.require_device(x, fn="quantize_nvfp4")
    # The kernel works in float64 as the reference's x.to(float64); fp32 / bf16 / fp16 / fp64 are read
    # as they are, any other real dtype is widened to float64 first (exact below 2**53).
    xx = x if x.dtype in (torch.float32, torch.bfloat16, torch.float16, torch.float64) else x.to(torch.float64)
    xx = xx.contiguous()
    dt = _lib.DTYPE_F64 if xx.dtype == torch.float64 else _lib.sqx_dtype(xx.dtype)
    packed = torch.empty(rows, k // 2, dtype=torch.uint8, device=dev)
    scales = torch.empty(rows, k // SF_VEC_SIZE, dtype=torch.uint8, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        _lib.check(_lib.load().sqx_nvfp4_ceil_quantize(xx.data_ptr(), dt, rows, k,
                                                       packed.data_ptr(), scales.data_ptr(), status.data_ptr(),
                                                       _stream(xx)), "quantize_nvfp4")
    _raise_on(status, "quantize_nvfp4")
    return NVFP4Operand(packed, scales, rows, k)


def dequantize_nvfp4(op: NVFP4Operand, dtype: torch.dtype = torch.float32) -> Tensor:
    """NVFP4 -> ``[rows, k]`` (b_r6.py:228-244): code value times block scale, exact in fp32 and in
    bf16 (``dtype``)."""
    if dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"dequantize_nvfp4 writes float32 or bfloat16, got {dtype}")
    dev = _lib.require_device(op.packed, op.scales, fn="dequantize_nvfp4")
    out = torch.empty(op.rows, op.k, dtype=dtype, device=dev)
    with torch.cuda.device(dev):
        _lib.check(_lib.load().sqx_nvfp4_ceil_dequantize(op.packed.contiguous().data_ptr(),
                                                         op.scales.contiguous().data_ptr(), op.rows, op.k,
                                                         out.data_ptr(), _lib.sqx_dtype(dtype), _stream(out)),
                   "dequantize_nvfp4")
    return out


_tiles = _device.TensorKeyedCache()


def _tiled(op: NVFP4Operand) -> FP4Tiled:
    def build() -> FP4Tiled:
        lib = _lib.load()
        dev = op.packed.device
        wt = torch.empty(lib.sqx_fp4_tiled_weight_bytes(op.rows, op.k), dtype=torch.uint8, device=dev)
        st = torch.empty(lib.sqx_fp4_tiled_scale_bytes(op.rows, op.k, _lib.FP4_NV), dtype=torch.uint8, device=dev)
        with torch.cuda.device(dev):
            _lib.check(lib.sqx_fp4_tile(op.packed.contiguous().data_ptr(), 1, op.scales.contiguous().data_ptr(),
                                        _lib.FP4_SCALE_NV_E4M3, SF_VEC_SIZE, op.rows, op.k, wt.data_ptr(),
                                        st.data_ptr(), _stream(wt)), "b_r6_gemm_packed (tile)")
        return FP4Tiled(wt, st, _lib.FP4_NV, torch.ones((), dtype=torch.float32, device=dev), op.rows, op.k)

    return _tiles.get((op.packed, op.scales), (op.rows, op.k), build)


def b_r6_gemm_packed(a: NVFP4Operand, b: NVFP4Operand) -> Tensor:
    """``C = A @ B.T`` for two quantized operands (``b`` is ``[N, K]``), fp32 accumulation, fp32
    result (b_r6.py:251-275)."""
    if a.k != b.k:
        raise ValueError(f"b_r6_gemm_packed inner dimensions disagree: {a.k} vs {b.k}")
    _lib.require_device(a.packed, b.packed, fn="b_r6_gemm_packed")
    xa = dequantize_nvfp4(a, torch.bfloat16)  # exact
    return fp4_linear_tiled(xa, _tiled(b), out_dtype=torch.float32)


def b_r6_gemm(a: Tensor, b: Tensor) -> Tensor:
    """``C = A @ B`` for real ``a [M, K]`` and ``b [K, N]``, both quantized to NVFP4 first
    (b_r6.py:278-303)."""
    if a.dtype not in (torch.bfloat16, torch.float32) or b.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"b_r6_gemm quantizes its operands to NVFP4, so it takes a real dtype it can round "
                        f"(bfloat16 or float32), got {a.dtype} and {b.dtype}. Already-quantized operands go "
                        f"to b_r6_gemm_packed")
    if a.ndim != 2 or b.ndim != 2:
        raise ValueError(f"b_r6_gemm expects 2-D operands, got {a.ndim}-D and {b.ndim}-D")
    if a.shape[1] != b.shape[0]:
        raise ValueError(f"b_r6_gemm inner dimensions disagree: {a.shape[1]} vs {b.shape[0]}")
    return b_r6_gemm_packed(quantize_nvfp4(a), quantize_nvfp4(b.t().contiguous()))


def reference_gemm(a: Tensor, b: Tensor) -> Tensor:
    """The reference's correctness problem (b_r6.py:306-331): quantize both operands, dequantize, and
    multiply with fp32 accumulation — on this build's kernels the same computation as
    :func:`b_r6_gemm` (exact products of the dequantized operands, fp32 sums)."""
    return b_r6_gemm(a.float() if a.dtype != torch.float32 else a, b.float() if b.dtype != torch.float32 else b)


def _elementwise(values: Tensor, fn: str, divisor: float | None):
    dev = _lib.require_device(values, fn=fn)
    v = values.to(torch.float64).contiguous().reshape(-1)
    codes = torch.empty(v.shape, dtype=torch.uint8, device=dev)
    out = torch.empty(v.shape, dtype=torch.float64, device=dev) if divisor is not None else None
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    lib = _lib.load()
    with torch.cuda.device(dev):
        if divisor is None:
            rc = lib.sqx_e2m1_round_rne(v.data_ptr(), v.numel(), codes.data_ptr(), status.data_ptr(), _stream(v))
        else:
            rc = lib.sqx_ue4m3_ceil(v.data_ptr(), v.numel(), float(divisor), codes.data_ptr(), out.data_ptr(),
                                    status.data_ptr(), _stream(v))
    _lib.check(rc, fn)
    st = int(status.item())
    if st & _NON_FINITE:
        if divisor is None:
            raise ValueError(f"{fn}: E2M1 encodes neither NaN nor Inf (NanInfEncoding::NONE) — a non-finite input "
                             "cannot be represented and must be rejected, not saturated")
        raise ValueError(f"{fn}: not a finite non-negative magnitude")
    if st & _RANGE:
        raise ValueError(f"{fn}: a value exceeds UE4M3's maximum {UE4M3_MAX:g}; unrepresentable")
    shape = values.shape
    return codes.reshape(shape), (None if out is None else out.reshape(shape))


def ue4m3_ceil_code(values: Tensor) -> Tensor:
    """Smallest UE4M3 code whose value is ``>= v``, elementwise (nvfp4_layout.py:341-363)."""
    return _elementwise(values, "ue4m3_ceil_code", 1.0)[0]


def scale_for_amax(amax: Tensor) -> tuple[Tensor, Tensor]:
    """``amax -> (UE4M3 code, its value as float64)`` of ``ceil_ue4m3(amax / 6)``, elementwise;
    amax 0 gives code 0 and scale 0 (nvfp4_layout.py:366-387)."""
    return _elementwise(amax, "scale_for_amax", E2M1_MAX)


def e2m1_round_code(values: Tensor) -> Tensor:
    """Nearest E2M1 code of already-scaled values, ties to even, saturating at ±6, with the sign bit
    set for every negative value (nvfp4_layout.py:390-416: ``code = 8 if value < 0``, so -0.2 gives
    0x8 and -0.0 gives 0x0). ``quantize_nvfp4`` instead stores a value that rounds to zero as +0
    (b_r6.py:217-223)."""
    return _elementwise(values, "e2m1_round_code", None)[0]
