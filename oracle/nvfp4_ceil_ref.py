"""numpy restatement of scratch_llm's second NVFP4 convention (the b_r6 kernel rung's operands) —
TEST INFRASTRUCTURE ONLY: imported by tests/ and nowhere in the product package.

The reference quantizes a real ``[rows, k]`` operand in blocks of ``SF_VEC_SIZE = 16`` along k
(src/scratch_llm/kernels/gemm/cuda/b_r6.py:155-215, with the scalar rules of
src/scratch_llm/kernels/gemm/nvfp4_layout.py:341-416):
  * float64 throughout: ``amax = max |x|`` per block;
  * ``scale = ceil_ue4m3(amax / 6)``: the smallest unsigned-E4M3 value (bias 7, subnormals m * 2**-9,
    maximum 448 at code 0x7E, 0x7F is NaN) that is >= amax / 6; amax / 6 > 448 raises; an all-zero
    block gets code 0 (scale 0) and divides by 1;
  * ``y = x / scale`` in float64, then the nearest E2M1 magnitude (0, .5, 1, 1.5, 2, 3, 4, 6) with
    ties to the even magnitude index (5 -> 4, 0.75 -> 1, 0.25 -> 0), saturating at 6;
  * in the quantizer, the sign bit only for a non-zero magnitude (zero is always code 0x0,
    b_r6.py:217-223); the scalar helper ``e2m1_round_code`` (nvfp4_layout.py:390-416) sets it for
    every negative input instead, so -0.2 gives 0x8;
  * two codes per byte, the lower k in the low nibble; NaN or Inf anywhere raises.
No global scale. The reference stores the scale bytes in the CUTLASS tile swizzle; here (and in
the build) they are a row-major ``[rows, k/16]`` uint8 array of UE4M3 codes, the build's own layout.

Pinning (tests/test_oracle_nvfp4_ceil.py): the reference test's tie table
(tests/kernels/gemm/test_k1_b_r6.py:452-469) and ceil-scale theorem and tightness checks (:472-500),
the round-trip bound and idempotence (:517-561), zero blocks, non-finite refusal and nibble order
(:564-611); independently, the UE4M3 ceiling against torch's ``float8_e4m3fn`` cast (the same
grid, round to nearest even) and the E2M1 rounding against a brute-force nearest search; the two
sign rules by code-byte known answers read off nvfp4_layout.py:399-416 and b_r6.py:217-223
(tests/golden/known_answers.json, ``e2m1_round_code_scalar``).
"""

from __future__ import annotations

import numpy as np

SF_VEC_SIZE = 16  # nvfp4_layout.py:149
E2M1_MAGNITUDES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)  # nvfp4_layout.py:306-307
E2M1_MAX = 6.0  # :310
E2M1_UNIT_ROUNDOFF = 0.25  # :318
UE4M3_CEIL_RELATIVE = 0.125  # :323
UE4M3_MAX = 448.0
UE4M3_MIN_POSITIVE = 2.0**-9
UE4M3_MIN_NORMAL = 2.0**-6


def ue4m3_value(code) -> np.ndarray:
    """Unsigned E4M3 decode (4 exponent bits, bias 7, 3 mantissa bits; 0x7F is NaN), float64."""
    c = np.asarray(code, np.int64) & 0x7F
    e, m = c >> 3, c & 7
    v = np.where(e == 0, m * 2.0**-9, (1.0 + m / 8.0) * np.exp2(e.astype(np.float64) - 7.0))
    return np.where(c == 0x7F, np.nan, v)


_GRID_CODES = np.arange(0x7F, dtype=np.int64)  # every finite code, ascending in value
_GRID = ue4m3_value(_GRID_CODES)
assert np.all(np.diff(_GRID) > 0)


def ue4m3_ceil_code(v) -> np.ndarray:
    """nvfp4_layout.py:341-363 (b_r6.py:192-201 vectorized): the smallest code whose value is >= v."""
    v = np.asarray(v, np.float64)
    if not np.all(np.isfinite(v)) or np.any(v < 0):
        raise ValueError("ue4m3_ceil_code: not a finite non-negative magnitude")
    idx = np.searchsorted(_GRID, v, side="left")
    if np.any(idx >= _GRID.size):
        raise ValueError(f"ue4m3_ceil_code: {float(v.max())} exceeds UE4M3's maximum {UE4M3_MAX:g}")
    return _GRID_CODES[idx].astype(np.uint8)


def scale_for_amax(amax) -> tuple[np.ndarray, np.ndarray]:
    """nvfp4_layout.py:366-387: ``(code, value)`` of ``ceil_ue4m3(amax / 6)``; amax 0 gives (0, 0)."""
    a = np.asarray(amax, np.float64)
    if not np.all(np.isfinite(a)) or np.any(a < 0):
        raise ValueError("scale_for_amax: amax must be a finite non-negative magnitude")
    code = ue4m3_ceil_code(a / E2M1_MAX)
    code = np.where(a == 0.0, np.uint8(0), code).astype(np.uint8)
    return code, ue4m3_value(code)


_MIDS = np.array([0.5 * (E2M1_MAGNITUDES[i] + E2M1_MAGNITUDES[i + 1]) for i in range(7)])  # b_r6.py:123-128


def _e2m1_magnitude(y) -> np.ndarray:
    """nvfp4_layout.py:403-416 / b_r6.py:205-216: index of the nearest E2M1 magnitude, ties to the
    even index, saturating at 6 (index 7)."""
    a = np.abs(y)
    lo = np.searchsorted(_MIDS, a, side="left")  # ties round down
    hi = np.searchsorted(_MIDS, a, side="right")  # ties round up
    return np.where((hi > lo) & (lo % 2 == 1), hi, lo)


def e2m1_round_code(y) -> np.ndarray:
    """nvfp4_layout.py:390-416, the scalar helper: the magnitude index with the sign bit set for every
    ``y < 0`` (``code = 8 if value < 0 else 0``, :402), so a negative value that rounds to magnitude 0
    gives 0x8 while -0.0 (not below zero) gives 0x0."""
    y = np.asarray(y, np.float64)
    if not np.all(np.isfinite(y)):
        raise ValueError("e2m1_round_code: E2M1 encodes neither NaN nor Inf (NanInfEncoding::NONE)")
    return (_e2m1_magnitude(y) | np.where(y < 0, 8, 0)).astype(np.uint8)


def _e2m1_quant_code(y) -> np.ndarray:
    """b_r6.py:205-223, the quantizer's codes: the same magnitude, but the sign bit only on a non-zero
    magnitude (zero is stored as canonical +0)."""
    y = np.asarray(y, np.float64)
    mag = _e2m1_magnitude(y)
    return (mag | np.where((y < 0) & (mag > 0), 8, 0)).astype(np.uint8)


def e2m1_value(code) -> np.ndarray:
    c = np.asarray(code, np.int64)
    v = np.asarray(E2M1_MAGNITUDES, np.float64)[c & 7]
    return np.where(c & 8, -v, v)


def quantize(x) -> tuple[np.ndarray, np.ndarray]:
    """b_r6.py:155-225: ``x [rows, k]`` -> (packed uint8 ``[rows, k/2]``, scale codes uint8
    ``[rows, k/16]`` row-major)."""
    x = np.asarray(x)
    if x.ndim != 2:
        raise ValueError(f"quantize_nvfp4 expects a 2-D operand, got {x.ndim}-D")
    rows, k = x.shape
    if k % SF_VEC_SIZE:
        raise ValueError(f"quantize_nvfp4: K={k} is not a multiple of SF_VEC_SIZE={SF_VEC_SIZE}")
    xf = x.astype(np.float64)
    if not np.all(np.isfinite(xf)):
        raise ValueError("quantize_nvfp4: operand contains NaN or Inf")
    blocks = xf.reshape(rows, k // SF_VEC_SIZE, SF_VEC_SIZE)
    amax = np.abs(blocks).max(axis=-1)
    code, scale = scale_for_amax(amax)
    y = blocks / np.where(scale > 0, scale, 1.0)[..., None]
    codes = _e2m1_quant_code(y).reshape(rows, k)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    return packed, code.reshape(rows, k // SF_VEC_SIZE)


def dequantize(packed, scales) -> np.ndarray:
    """b_r6.py:228-244: fp32 ``code value * scale``, exact (at most 6 significant bits)."""
    packed = np.asarray(packed, np.uint8)
    rows, half = packed.shape
    codes = np.stack((packed & 0xF, packed >> 4), axis=-1).reshape(rows, 2 * half)
    vals = e2m1_value(codes).reshape(rows, -1, SF_VEC_SIZE) * ue4m3_value(scales)[..., None]
    return vals.reshape(rows, 2 * half).astype(np.float32)


def reference_gemm(a, b) -> np.ndarray:
    """b_r6.py:306-331: quantize a [M, K] and b [K, N] (b along its K, i.e. b.T's rows), dequantize,
    and multiply; returned in float64 (the reference's fp32 matmul is within fp32 accumulation of it)."""
    qa = dequantize(*quantize(np.asarray(a, np.float32)))
    qb = dequantize(*quantize(np.ascontiguousarray(np.asarray(b, np.float32).T)))
    return qa.astype(np.float64) @ qb.astype(np.float64).T
