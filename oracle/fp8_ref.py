"""numpy restatement of scratch_llm's FP8 E4M3 quantizers and W8A8 oracle — TEST INFRASTRUCTURE ONLY.

Restates src/scratch_llm/quant/fp8_weights.py (saturating_cast_e4m3 :117-124, _amax_scale :127-130,
quantize_per_channel :133-143, quantize_per_token :146-155, dequantize :158-160,
fp8_linear_reference :265-286) and fp8_kv_per_head.py (per_head_amax :77-85, per_head_scale :88-90,
quantize_per_head :93-96, dequantize_per_head :99-101, saturated_count :104-107).

Pinning (tests/test_oracle_fp8.py):
  e4m3_encode_sat ..... torch's own float8_e4m3fn cast after the clamp, over every code's value, every
                        midpoint between neighbouring codes (ties to even), their fp32 neighbours, a
                        dense log grid from 2**-12 to 1e6, +-0, infinities and NaN; the reference's
                        named values [448, 464, 465, 1e5] -> [448, 448, NaN, NaN] for the raw cast
                        (tests/quant/test_s1_s_r2.py:203-223)
  e4m3_decode ......... closed form over all 256 codes against torch's float8_e4m3fn -> float32
  quantize rows ....... the reference's laws: round trip within 2**-4 relative above 2**-6 and 2**-10
                        absolute below; each row's largest code is +-448; rows are independent
                        (tests/quant/test_s1_s_r2.py:134-200)
  per-head ............ flush below half the smallest subnormal, idempotence at a fixed scale,
                        saturation counted (tests/quant/test_s1_s_r2.py:278-348)
  fp8_linear_reference  the definition of a matmul, brute force (tests/quant/test_s1_s_r2.py:401-416)
"""

from __future__ import annotations

import numpy as np

F32 = np.float32
E4M3_MAX = F32(448.0)
MIN_SCALE = F32(1.0 / (448.0 * 512.0))

# value of every code (OCP e4m3fn: bias 7, subnormals m * 2**-9, NaN = S.1111.111)
_VALUES = np.zeros(256, dtype=np.float64)
for _c in range(256):
    _s, _e, _m = _c >> 7, (_c >> 3) & 15, _c & 7
    _v = _m * 2.0**-9 if _e == 0 else (1 + _m / 8) * 2.0 ** (_e - 7)
    _VALUES[_c] = np.nan if (_e == 15 and _m == 7) else (-_v if _s else _v)


def e4m3_decode(codes) -> np.ndarray:
    """Code bytes -> fp32 values."""
    return _VALUES[np.asarray(codes, dtype=np.uint8)].astype(F32)


def e4m3_encode_sat(v) -> np.ndarray:
    """saturating_cast_e4m3: clamp to +-448, then round to nearest (ties to the even code). NaN keeps
    its sign bit and becomes 0x7f / 0xff. Returns code bytes."""
    v = np.asarray(v, dtype=F32)
    sign = (np.signbit(v)).astype(np.uint8) << 7
    a = np.minimum(np.abs(v.astype(np.float64)), 448.0)
    # candidate codes 0..126 (positive, finite); pick nearest, ties to even code
    pos = _VALUES[:127]
    idx = np.searchsorted(pos, a, side="left")
    idx = np.clip(idx, 1, 126)
    lo, hi = pos[idx - 1], pos[idx]
    d_lo, d_hi = a - lo, hi - a
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (idx % 2 == 0))
    code = np.where(pick_hi, idx, idx - 1).astype(np.uint8)
    code = np.where(a <= 0.0, 0, code).astype(np.uint8)
    out = (code | sign).astype(np.uint8)
    return np.where(np.isnan(v), sign | 0x7F, out).astype(np.uint8)


def _nan_amax(x: np.ndarray, axis) -> np.ndarray:
    a = np.abs(x.astype(F32))
    m = np.max(a, axis=axis, keepdims=True)
    return np.where(np.isnan(a).any(axis=axis, keepdims=True), np.float32(np.nan), m).astype(F32)


def _scale_from_amax(amax: np.ndarray) -> np.ndarray:
    q = (amax.astype(F32) / E4M3_MAX).astype(F32)
    return np.where(np.isnan(q), q, np.maximum(q, MIN_SCALE)).astype(F32)


def quantize_rows(x) -> tuple[np.ndarray, np.ndarray]:
    """quantize_per_channel / quantize_per_token of a 2-D array: (codes [R, C], scale [R, 1] fp32)."""
    x = np.asarray(x, dtype=F32)
    s = _scale_from_amax(_nan_amax(x, axis=1))
    return e4m3_encode_sat((x / s).astype(F32)), s


def dequantize(codes, scale) -> np.ndarray:
    return (e4m3_decode(codes) * np.asarray(scale, dtype=F32)).astype(F32)


def fp8_linear_reference(x, w_codes, w_scale, bias=None) -> np.ndarray:
    """fp8_linear_reference in float64: x quantized per token, both operands dequantized exactly."""
    xc, xs = quantize_rows(x)
    xd = e4m3_decode(xc).astype(np.float64) * xs.astype(np.float64)
    wd = e4m3_decode(w_codes).astype(np.float64) * np.asarray(w_scale, dtype=np.float64).reshape(-1, 1)
    out = xd @ wd.T
    if bias is not None:
        out = out + np.asarray(bias, dtype=np.float64)
    return out


def per_head_amax(x) -> np.ndarray:
    """(B, H, T, D) -> (1, H, 1, 1) fp32."""
    return _nan_amax(np.asarray(x, dtype=F32), axis=(0, 2, 3))


def per_head_scale(x) -> np.ndarray:
    return _scale_from_amax(per_head_amax(x))


def quantize_per_head(x, scale) -> np.ndarray:
    return e4m3_encode_sat((np.asarray(x, dtype=F32) / np.asarray(scale, dtype=F32)).astype(F32))


def dequantize_per_head(codes, scale) -> np.ndarray:
    return dequantize(codes, scale)


def saturated_count(x, scale) -> int:
    return int((np.abs(np.asarray(x, dtype=F32)) > (E4M3_MAX * np.asarray(scale, dtype=F32)).astype(F32)).sum())
