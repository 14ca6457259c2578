"""numpy restatement of scratch_llm's quant arithmetic — TEST INFRASTRUCTURE ONLY (see package doc).

Every function cites the reference file:line it restates. Arithmetic is fp32 wherever the
reference computes in fp32 (numpy float32 division is IEEE round-to-nearest, ``np.rint`` rounds
half to even exactly like ``torch.round``), so quantize/pack results are meant to be bit-identical.
Linears return float64 results of the reference's *inputs to the GEMM* (the dequantized weight
after its cast to the activation dtype), which tests round or compare within a tolerance.

Pinning (how each function is checked against the reference, in tests/test_oracle_*.py):
  pack_int4 / unpack_int4 ........ reference known answers (0x12, 0x78, 0xFF, odd length) + closed form
  quantize_groupwise_int4 ......... half-even tie vectors, code range, recorded SQNR 18.64 dB
                                    (bench/RESULTS.md:560) on the reference test's seeded data
  dequantize_groupwise_int4 ....... exact products (closed form)
  w4a16_linear .................... float64 brute force on tiny shapes; reference rel-MSE law
  quantize_symmetric / affine ..... book vector [1.2,-0.8,2.5,-1.7] -> [61,-41,127,-86]; zero exact;
                                    recorded SQNRs (bench/RESULTS.md:558-559)
  w8a8_linear ..................... exact integer accumulation vs brute force; rel err < 1.5e-2 law
  quantize_awq_int4 ............... alpha=0 identity with naive int4; linear == x @ awq_dequantize.T
  search_awq_scale ................ reference laws (AWQ beats naive > 1.4x, interior alpha);
                                    exact alpha choice parity unpinned (torch reduction order)
  e2m1_round_to_code / decode ..... grid self-map, saturation, [1.7,2.4,4.9,5.1] -> [1.5,2,4,6],
                                    golden vectors for ties, huge values, infinities and NaN
  pack_fp4 / unpack_fp4 ........... checkpoint named bytes 0x80/0x7F/0x21 (tests/test_k3_checkpoint.py:281-292)
  quantize_e4m3 ................... self-map + saturation known answers, exhaustive vs torch.float8_e4m3fn
  quantize_e8m0 ................... powers-of-two self-map; golden vectors at binade midpoints
  e8m0_no_overflow_scale .......... golden vectors from the reference at powers of two (911 cases):
                                    ceil of the correctly rounded fp32 log2 (tests/golden)
  nvfp4 / mxfp4 quantize .......... NVFP4 MSE < MXFP4 law; recorded 20.43 / 18.74 dB (bench/RESULTS.md:561)
  quant_linear_nvfp4 .............. == dequant-matmul within 1e-4 (law at tests/test_quant_nvfp4_mxfp4.py:183-193)
  dequantize_mxfp4 (checkpoint) ... bit-level decoder over all 256 bytes x scale codes
"""

from __future__ import annotations

import math

import numpy as np

F32 = np.float32
FLT_MIN = np.float32(np.finfo(np.float32).tiny)

# ================================================================================================
# bf16 / fp16 rounding helpers (what `.to(torch.bfloat16)` / `.to(torch.float16)` do to fp32 values)
# ================================================================================================


def bf16_bits(a) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even (NaN kept quiet)."""
    u = np.asarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x007FFFFF) != 0)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def bf16_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(a) -> np.ndarray:
    """fp32 values rounded to the nearest bf16, returned as fp32."""
    return bf16_to_f32(bf16_bits(a))


def round_to(a, dtype: str) -> np.ndarray:
    """Round fp32 values to the activation dtype ('bf16', 'f16' or 'f32'), returned as fp32."""
    a = np.asarray(a, dtype=np.float32)
    if dtype == "bf16":
        return round_bf16(a)
    if dtype == "f16":
        return a.astype(np.float16).astype(np.float32)
    return a


# ================================================================================================
# INT4 group-wise (src/scratch_llm/quant/int4_group.py)
# ================================================================================================
GROUP_SIZE = 128  # int4_group.py:54
INT4_QMIN = -8  # int4_group.py:55
INT4_QMAX = 7  # int4_group.py:56


def pack_int4(q) -> np.ndarray:
    """int4_group.py:62-82 — two signed nibbles per byte, element 2i in the high nibble."""
    q = np.asarray(q)
    if q.ndim != 1:
        raise ValueError(f"pack_int4 expects a 1-D tensor, got shape {tuple(q.shape)}")
    nib = q.astype(np.int64) & 0xF
    if nib.size % 2:
        nib = np.concatenate([nib, np.zeros(1, np.int64)])
    return ((nib[0::2] << 4) | nib[1::2]).astype(np.uint8)


def unpack_int4(packed, n: int) -> np.ndarray:
    """int4_group.py:85-102 — high nibble first; sign-extend each nibble; first n values."""
    b = np.asarray(packed)
    if b.ndim != 1:
        raise ValueError(f"unpack_int4 expects a 1-D tensor, got shape {tuple(b.shape)}")
    b = b.astype(np.int64)
    both = np.empty(2 * b.size, dtype=np.int64)
    both[0::2] = (b >> 4) & 0xF
    both[1::2] = b & 0xF
    both = both[:n]
    return np.where(both >= 8, both - 16, both).astype(np.int8)


def quantize_groupwise_int4(w, group_size: int = GROUP_SIZE) -> tuple[np.ndarray, np.ndarray]:
    """int4_group.py:108-129 — s = max(absmax/7, FLT_MIN) (fp32), q = clamp(rint(w/s), -8, 7)."""
    w = np.asarray(w)
    if w.ndim != 2:
        raise ValueError(f"expected a 2-D weight, got shape {tuple(w.shape)}")
    rows, cols = w.shape
    if cols % group_size != 0:
        raise ValueError(f"in_features={cols} not divisible by group_size={group_size}")
    g = cols // group_size
    wf = w.astype(np.float32).reshape(rows, g, group_size)
    absmax = np.abs(wf).max(axis=-1, keepdims=True)
    s = absmax / F32(INT4_QMAX)
    s = np.where(s < FLT_MIN, FLT_MIN, s).astype(np.float32)
    with np.errstate(invalid="ignore"):
        q = np.clip(np.rint(wf / s), INT4_QMIN, INT4_QMAX)
    q = np.nan_to_num(q, nan=0.0).astype(np.int8)
    return q.reshape(rows, cols), s.reshape(rows, g)


def dequantize_groupwise_int4(q, scales, group_size: int = GROUP_SIZE) -> np.ndarray:
    """int4_group.py:132-142 — fp32 q * s."""
    q = np.asarray(q)
    rows, cols = q.shape
    g = cols // group_size
    qf = q.astype(np.float32).reshape(rows, g, group_size)
    return (qf * np.asarray(scales, np.float32).reshape(rows, g, 1)).reshape(rows, cols)


def linear_f64(x, w_eff, bias=None) -> np.ndarray:
    """float64 ``x @ w_eff.T (+ bias)`` — the exact value a GEMM on these operands approximates."""
    x64 = np.asarray(x, np.float64)
    y = x64.reshape(-1, x64.shape[-1]) @ np.asarray(w_eff, np.float64).T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    return y.reshape(*x64.shape[:-1], y.shape[-1])


def w4a16_linear(x, q, scales, bias=None, group_size: int = GROUP_SIZE, act: str = "bf16") -> np.ndarray:
    """int4_group.py:148-164 — F.linear(x, dequant(q, s).to(x.dtype), bias), in float64.

    ``x`` holds values already representable in ``act``; the weight is rounded to ``act`` first,
    as the reference's ``.to(x.dtype)`` does. Returns the float64 product (not yet rounded)."""
    w_eff = round_to(dequantize_groupwise_int4(q, scales, group_size), act)
    return linear_f64(x, w_eff, bias)


def sqnr_db(ref, approx) -> float:
    """int4_group.py:170-177 / int8.py:81-90 — 10*log10(sum ref^2 / sum (ref-approx)^2), float64."""
    r = np.asarray(ref, np.float64)
    a = np.asarray(approx, np.float64)
    noise = float(((r - a) ** 2).sum())
    if noise == 0.0:
        return float("inf")
    return float(10.0 * math.log10(float((r**2).sum()) / noise))


def mse(ref, approx) -> float:
    """int4_group.py:180-183 — float64 mean squared error."""
    return float(((np.asarray(ref, np.float64) - np.asarray(approx, np.float64)) ** 2).mean())


# ------------------------------------------------------------------------------------------------
# Asymmetric uint4 (build-defined: no reference symbol — parity unpinned by the
# reference). The 4-bit analogue of quantize_affine (int8.py:142-172) applied per group.
# ------------------------------------------------------------------------------------------------
def quantize_groupwise_uint4_asym(w, group_size: int = GROUP_SIZE, param: str = "bf16"):
    """Per group: lo = min(min(w), 0), hi = max(max(w), 0); s = max((hi-lo)/15, 1e-12);
    z = clamp(rint(-lo/s), 0, 15) (a zero zero-point is +0); q = clamp(rint(w/s + z), 0, 15). With
    ``param='bf16'`` the scale is rounded to bf16 *before* codes are computed, so the stored (s, z)
    reproduce the codes. Pinned by its invariants (zero exact, error <= s/2 in range), not by any
    reference symbol."""
    w = np.asarray(w)
    rows, cols = w.shape
    if cols % group_size != 0:
        raise ValueError(f"in_features={cols} not divisible by group_size={group_size}")
    g = cols // group_size
    wf = w.astype(np.float32).reshape(rows, g, group_size)
    lo = np.minimum(wf.min(axis=-1, keepdims=True), F32(0))
    hi = np.maximum(wf.max(axis=-1, keepdims=True), F32(0))
    s = (hi - lo) / F32(15)
    s = np.where(s < F32(1e-12), F32(1e-12), s).astype(np.float32)
    if param == "bf16":
        s = round_bf16(s)
    z = (np.clip(np.rint(-lo / s), 0, 15) + F32(0)).astype(np.float32)  # +0, never -0, for zero groups
    q = np.clip(np.rint(wf / s + z), 0, 15).astype(np.int8)
    return q.reshape(rows, cols), s.reshape(rows, g), z.reshape(rows, g)


def dequantize_groupwise_uint4_asym(q, scales, zeros, group_size: int = GROUP_SIZE) -> np.ndarray:
    q = np.asarray(q)
    rows, cols = q.shape
    g = cols // group_size
    qf = q.astype(np.float32).reshape(rows, g, group_size)
    s = np.asarray(scales, np.float32).reshape(rows, g, 1)
    z = np.asarray(zeros, np.float32).reshape(rows, g, 1)
    return ((qf - z) * s).reshape(rows, cols)


# ================================================================================================
# INT8 (src/scratch_llm/quant/int8.py)
# ================================================================================================
_SYM_QMAX = 127  # int8.py:75
_AFF_QMAX = 255  # int8.py:78


def _reduce_keep(x: np.ndarray, axis, fn):
    if axis is None:
        return fn(x)
    dims = tuple(d for d in range(x.ndim) if d != axis)
    return fn(x, axis=dims, keepdims=True)


def quantize_symmetric(x, axis=None, eps: float = 1e-12, dtype: str = "f32"):
    """int8.py:102-125 — computed in x's dtype (``dtype`` 'f32', 'bf16' or 'f16'; x holds values of
    that dtype): s = max(rd(amax / 127), rd(eps)), q = clamp(rint(rd(x / s)), -127, 127), where rd
    rounds an fp32 result to the dtype exactly where torch does. axis = the kept dim (keepdim)."""
    xf = round_to(np.asarray(x, np.float32), dtype)
    amax = np.asarray(_reduce_keep(np.abs(xf), axis, np.max), np.float32)
    s = round_to(amax / F32(_SYM_QMAX), dtype)
    e = round_to(np.float32(eps), dtype)
    s = np.where(s < e, e, s).astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        q = np.clip(np.rint(round_to(xf / s, dtype)), -_SYM_QMAX, _SYM_QMAX)
    return np.nan_to_num(q).astype(np.int8), s


def dequantize_symmetric(q, s, dtype: str = "f32") -> np.ndarray:
    """int8.py:127-129 — q.to(s.dtype) * s, rounded to the scale dtype."""
    return round_to(np.asarray(q).astype(np.float32) * np.asarray(s, np.float32), dtype)


def quantize_affine(x, axis=None, eps: float = 1e-12, dtype: str = "f32"):
    """int8.py:141-171 — in x's dtype: lo = min(min(x), 0), hi = max(max(x), 0);
    s = max(rd(rd(hi - lo) / 255), rd(eps)); z = clamp(rint(rd(-lo / s)), 0, 255);
    q = clamp(rint(rd(rd(x / s) + z)), 0, 255)."""
    xf = round_to(np.asarray(x, np.float32), dtype)
    xmin = np.minimum(np.asarray(_reduce_keep(xf, axis, np.min), np.float32), F32(0))
    xmax = np.maximum(np.asarray(_reduce_keep(xf, axis, np.max), np.float32), F32(0))
    s = round_to(round_to(xmax - xmin, dtype) / F32(_AFF_QMAX), dtype)
    e = round_to(np.float32(eps), dtype)
    s = np.where(s < e, e, s).astype(np.float32)
    z = np.clip(np.rint(round_to(-xmin / s, dtype)), 0, _AFF_QMAX).astype(np.float32)
    with np.errstate(invalid="ignore"):
        q = np.clip(np.rint(round_to(round_to(xf / s, dtype) + z, dtype)), 0, _AFF_QMAX)
    return np.nan_to_num(q).astype(np.uint8), s, z


def dequantize_affine(q, s, z, dtype: str = "f32") -> np.ndarray:
    """int8.py:174-176 — (q.to(s.dtype) - z) * s, each step rounded to the scale dtype."""
    qf = np.asarray(q).astype(np.float32)
    return round_to(round_to(qf - np.asarray(z, np.float32), dtype) * np.asarray(s, np.float32), dtype)


def w8a8_linear(x, w, dtype: str = "f32") -> np.ndarray:
    """int8.py:188-213 — per-token int8 x, per-row int8 w, exact integer accumulate, fp32 epilogue
    acc.to(fp32) * (s_x * s_w) with the scale product in the scales' dtype."""
    xf = np.asarray(x, np.float32)
    k = xf.shape[-1]
    x2 = xf.reshape(-1, k)
    qx, sx = quantize_symmetric(x2, axis=0, dtype=dtype)
    qw, sw = quantize_symmetric(np.asarray(w, np.float32), axis=0, dtype=dtype)
    acc = qx.astype(np.int64) @ qw.astype(np.int64).T
    y = acc.astype(np.float32) * round_to(sx * sw.reshape(1, -1), dtype)
    return y.reshape(*xf.shape[:-1], np.asarray(w).shape[0])


def int8_weight_linear(x, q, s, bias=None, act: str = "bf16") -> np.ndarray:
    """BASELINE config 1 (composition of int8.py:101-129 and F.linear): x @ (q*s).to(act).T, float64."""
    w_eff = round_to(dequantize_symmetric(q, np.asarray(s, np.float32).reshape(-1, 1)), act)
    return linear_f64(x, w_eff, bias)


# ================================================================================================
# AWQ (src/scratch_llm/quant/awq.py)
# ================================================================================================
def act_scale(x) -> np.ndarray:
    """awq.py:94-101 — per-input-channel mean |x| in fp32."""
    xf = np.abs(np.asarray(x, np.float32))
    return xf.reshape(-1, xf.shape[-1]).mean(axis=0, dtype=np.float32)


def normalize_scale(s) -> np.ndarray:
    """awq.py:104-112 — s.clamp_min(1e-4) / sqrt(max*min)."""
    s = np.asarray(s, np.float32)
    s = np.where(s < F32(1e-4), F32(1e-4), s).astype(np.float32)
    return (s / np.sqrt(F32(s.max()) * F32(s.min()))).astype(np.float32)


def quantize_awq_int4(w, chan_scale, group_size: int = GROUP_SIZE):
    """awq.py:154-175 (chan_scale branch) — group-int4 codes of w * s. Returns (q, group_scales, s)."""
    s = np.asarray(chan_scale, np.float32)
    w_scaled = np.asarray(w, np.float32) * s[None, :]
    q, gs = quantize_groupwise_int4(w_scaled, group_size)
    return q, gs, s


def awq_dequantize(q, group_scales, chan_scale, group_size: int = GROUP_SIZE) -> np.ndarray:
    """awq.py:178-181 — dequant(q, gs) / s (fp32 division)."""
    return dequantize_groupwise_int4(q, group_scales, group_size) / np.asarray(chan_scale, np.float32)[None, :]


def awq_linear(x, q, group_scales, chan_scale, bias=None, group_size: int = GROUP_SIZE, act: str = "bf16"):
    """awq.py:184-192 — F.linear(x, awq_dequantize(...).to(x.dtype), bias), float64."""
    w_eff = round_to(awq_dequantize(q, group_scales, chan_scale, group_size), act)
    return linear_f64(x, w_eff, bias)


def search_awq_scale(w, x, group_size: int = GROUP_SIZE, grid: int = 20):
    """awq.py:122-151 — alpha grid search on calibration output MSE. Returns (chan_scale, ratio, mse).

    fp32 arithmetic like the reference; reductions may sum in a different order than torch, so the
    chosen ratio can differ at near-ties (parity of the exact choice is unpinned)."""
    wf = np.asarray(w, np.float32)
    xf = np.asarray(x, np.float32).reshape(-1, wf.shape[1])
    y_ref = xf @ wf.T
    a = act_scale(xf)
    best = None
    for i in range(grid + 1):
        ratio = i / grid
        s = normalize_scale(np.power(a, F32(ratio)).astype(np.float32))
        q, gs = quantize_groupwise_int4(wf * s[None, :], group_size)
        w_eff = dequantize_groupwise_int4(q, gs, group_size) / s[None, :]
        cur = mse(y_ref, xf @ w_eff.T)
        if best is None or cur < best[2]:
            best = (s, ratio, cur)
    return best


# ================================================================================================
# FP4 E2M1, NVFP4, MXFP4 (src/scratch_llm/quant/nvfp4_mxfp4.py)
# ================================================================================================
FP4_MAGNITUDES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)  # nvfp4_mxfp4.py:65
E4M3_MAX = 448.0  # nvfp4_mxfp4.py:69
_FP4_MAX = 6.0
_TINY = 1e-30
_MAGS = np.array(FP4_MAGNITUDES, dtype=np.float32)


def e2m1_round_to_code(x) -> np.ndarray:
    """nvfp4_mxfp4.py:85-98 — index of the nearest E2M1 magnitude by fp32 distance |a - m|, the first
    index on ties (torch.argmin), a NaN input giving index 0; sign bit = x < 0 (so -0 keeps no sign
    bit, small negatives keep it). Distances are fp32, so inputs above ~2**25 tie at every anchor and
    infinities and huge values map to magnitude index 0, exactly as the reference does."""
    xf = np.asarray(x, np.float32)
    a = np.abs(xf)
    with np.errstate(invalid="ignore", over="ignore"):
        dist = np.abs(a[..., None] - _MAGS).astype(np.float32)
    idx = np.argmin(dist, axis=-1).astype(np.uint8)  # first minimum; a NaN row gives index 0
    idx = np.where(np.isnan(a), np.uint8(0), idx)
    sign = (xf < 0).astype(np.uint8)
    return (sign << 3) | idx


def e2m1_decode(code) -> np.ndarray:
    """nvfp4_mxfp4.py:101-106 — +-FP4_MAGNITUDES[code & 7] (code 8 decodes to -0.0)."""
    c = np.asarray(code).astype(np.int64)
    sign = np.where((c & 8) != 0, F32(-1.0), F32(1.0))
    return (sign * _MAGS[c & 7]).astype(np.float32)


def pack_fp4(codes) -> np.ndarray:
    """nvfp4_mxfp4.py:109-120 — element 2i in the LOW nibble; odd length padded with a zero code."""
    c = np.asarray(codes).astype(np.uint8).reshape(-1)
    if c.size % 2:
        c = np.concatenate([c, np.zeros(1, np.uint8)])
    return ((c[0::2] & 0xF) | ((c[1::2] & 0xF) << 4)).astype(np.uint8)


def unpack_fp4(packed, n: int) -> np.ndarray:
    """nvfp4_mxfp4.py:123-129."""
    p = np.asarray(packed).astype(np.uint8).reshape(-1)
    out = np.empty(2 * p.size, np.uint8)
    out[0::2] = p & 0xF
    out[1::2] = (p >> 4) & 0xF
    return out[:n]


def quantize_e4m3(v) -> np.ndarray:
    """nvfp4_mxfp4.py:135-147 — nearest E4M3 value (3 mantissa bits, exponent clamped to [-6, 8],
    round half to even, saturating at 448; non-positive -> 0). Computed as the closed form: the
    binade exponent of a positive fp32 is exact from its bit pattern."""
    vf = np.clip(np.asarray(v, np.float32), 0.0, E4M3_MAX).astype(np.float32)
    pos = vf > 0
    safe = np.where(pos, vf, F32(1.0))
    e = (safe.view(np.uint32) >> 23).astype(np.int64) - 127  # floor(log2) for normals
    sub = (safe.view(np.uint32) >> 23) == 0  # fp32 subnormals (far below the E4M3 range)
    e = np.where(sub, -127, e)
    e = np.clip(e, -6, 8)
    step = np.ldexp(np.float32(1.0), (e - 3).astype(np.int32)).astype(np.float32)
    q = (np.rint(safe / step) * step).astype(np.float32)
    q = np.clip(q, 0.0, E4M3_MAX).astype(np.float32)
    return np.where(pos, q, F32(0.0)).astype(np.float32)


def ceil_log2_exact(v) -> np.ndarray:
    """Exact ceil(log2(v)) for positive finite fp32 v, from the bit pattern."""
    vf = np.asarray(v, np.float32)
    u = vf.view(np.uint32).astype(np.int64)
    e = (u >> 23) - 127
    m = u & 0x7FFFFF
    # subnormals: normalise
    sub = (u >> 23) == 0
    if np.any(sub):
        mm = np.where(sub, m, 1)
        msb = np.floor(np.log2(mm.astype(np.float64))).astype(np.int64)
        e = np.where(sub, msb - 149, e)
        m = np.where(sub, mm - (np.int64(1) << msb), m)
    return e + (m != 0)


def log2_f32(v) -> np.ndarray:
    """fp32 log2 correctly rounded (float64 log2, then one rounding to fp32), the value torch's CPU
    log2 returns for fp32 inputs; pinned against the reference on 911 inputs near powers of two."""
    with np.errstate(divide="ignore"):
        return np.log2(np.asarray(v, np.float32).astype(np.float64)).astype(np.float32)


def e8m0_no_overflow_exponent(amax) -> np.ndarray:
    """nvfp4_mxfp4.py:162-174 — exponent of the MXFP4 block scale:
    clamp(ceil(log2(max(amax/6, 1e-30))), +-127) with log2 evaluated in fp32 (so amax/6 a few ulps
    above 2**k gives k when the fp32 log2 rounds down onto k)."""
    t = np.asarray(amax, np.float32) / F32(_FP4_MAX)
    t = np.where(t < F32(_TINY), F32(_TINY), t).astype(np.float32)
    return np.clip(np.ceil(log2_f32(t)), -127, 127).astype(np.int64)


def e8m0_no_overflow_scale(amax) -> np.ndarray:
    return np.ldexp(np.float32(1.0), e8m0_no_overflow_exponent(amax).astype(np.int32)).astype(np.float32)


def quantize_e8m0(v) -> np.ndarray:
    """nvfp4_mxfp4.py:150-159 — 2**clamp(rint(log2 v), +-127) with fp32 log2, 0 -> 0."""
    vf = np.asarray(v, np.float32)
    e = np.clip(np.rint(log2_f32(np.where(vf < F32(_TINY), F32(_TINY), vf))), -127, 127)
    return np.where(vf > 0, np.ldexp(np.float32(1.0), e.astype(np.int32)), F32(0.0)).astype(np.float32)


def _blockify(x, block: int):
    """nvfp4_mxfp4.py:180-187 — flatten row-major, zero-pad to a multiple of block."""
    flat = np.asarray(x, np.float32).reshape(-1)
    n = flat.size
    pad = (-n) % block
    if pad:
        flat = np.concatenate([flat, np.zeros(pad, np.float32)])
    return flat.reshape(-1, block), n


def nvfp4_quantize(x, block: int = 16):
    """nvfp4_mxfp4.py:212-223 — returns (codes (n_blocks, block) uint8, s_global f32, s_block f32, shape, n)."""
    xf = np.asarray(x, np.float32)
    xb, n = _blockify(xf, block)
    amax = np.abs(xb).max()
    s_global = np.float32(amax) / F32(E4M3_MAX * _FP4_MAX)
    s_global = np.float32(max(s_global, F32(_TINY)))
    block_amax = np.abs(xb).max(axis=1)
    s_block = quantize_e4m3((block_amax / F32(_FP4_MAX)) / s_global)
    scale = s_global * s_block
    scale = np.where(scale < F32(_TINY), F32(_TINY), scale).astype(np.float32)
    codes = e2m1_round_to_code(xb / scale[:, None])
    return codes, s_global, s_block, xf.shape, n


def nvfp4_dequantize(codes, s_global, s_block, shape, n) -> np.ndarray:
    """nvfp4_mxfp4.py:226-231."""
    mag = e2m1_decode(codes)
    scale = (np.float32(s_global) * np.asarray(s_block, np.float32))[:, None]
    return (mag * scale).reshape(-1)[:n].reshape(shape)


def mxfp4_quantize(x, block: int = 32, exponent=None):
    """nvfp4_mxfp4.py:257-265 — returns (codes (n_blocks, block) uint8, s_block f32, e8m0 bytes, shape, n).

    ``exponent`` optionally overrides the per-block scale exponent (used by tests that pin the
    reference's log2 rounding at powers of two)."""
    xf = np.asarray(x, np.float32)
    xb, n = _blockify(xf, block)
    block_amax = np.abs(xb).max(axis=1)
    e = e8m0_no_overflow_exponent(block_amax) if exponent is None else np.asarray(exponent)
    s_block = np.ldexp(np.float32(1.0), e.astype(np.int32)).astype(np.float32)
    s_block = np.where(s_block < F32(_TINY), F32(_TINY), s_block).astype(np.float32)
    codes = e2m1_round_to_code(xb / s_block[:, None])
    return codes, s_block, (e + 127).astype(np.uint8), xf.shape, n


def mxfp4_dequantize(codes, s_block, shape, n) -> np.ndarray:
    """nvfp4_mxfp4.py:268-272."""
    mag = e2m1_decode(codes)
    return (mag * np.asarray(s_block, np.float32)[:, None]).reshape(-1)[:n].reshape(shape)


def quant_linear_nvfp4_weight(weight, block: int = 16) -> np.ndarray:
    """nvfp4_mxfp4.py:307-322 — the dequantized NVFP4 weight quant_linear_nvfp4 multiplies by."""
    w = np.asarray(weight, np.float32)
    n_out, k = w.shape
    if k % block != 0:
        raise ValueError(f"K={k} must be a multiple of block={block} for the block-scaled GEMM")
    amax = np.abs(w).max()
    s_global = np.float32(max(np.float32(amax) / F32(E4M3_MAX * _FP4_MAX), F32(_TINY)))
    wb = w.reshape(n_out, k // block, block)
    block_amax = np.abs(wb).max(axis=2)
    s_block = quantize_e4m3((block_amax / F32(_FP4_MAX)) / s_global)
    scale = s_global * s_block
    scale = np.where(scale < F32(_TINY), F32(_TINY), scale).astype(np.float32)[..., None]
    codes = e2m1_round_to_code(wb / scale)
    return (e2m1_decode(codes) * scale).reshape(n_out, k).astype(np.float32)


def quant_linear_nvfp4(x, weight, block: int = 16) -> np.ndarray:
    """nvfp4_mxfp4.py:296-328 — y = x @ nvfp4(W).T with fp32 x, float64 here."""
    return linear_f64(np.asarray(x, np.float32), quant_linear_nvfp4_weight(weight, block))


# ================================================================================================
# On-disk MXFP4 (src/scratch_llm/k3/checkpoint.py:92-144)
# ================================================================================================
def dequantize_mxfp4_checkpoint(weight_packed, weight_scale) -> np.ndarray:
    """k3/checkpoint.py:92-144 — w[r,c] = E2M1(code[r,c]) * 2**(scale[r, c//32] - 127), float64, exact.
    Refuses non-uint8 halves, bad shapes and the NaN scale 0xFF with ValueError."""
    wp = np.asarray(weight_packed)
    ws = np.asarray(weight_scale)
    if wp.dtype != np.uint8 or ws.dtype != np.uint8:
        raise ValueError(f"MXFP4 halves must be uint8; got {wp.dtype}, {ws.dtype}")
    if wp.ndim != 2:
        raise ValueError(f"weight_packed must be [out, in/2]; got {tuple(wp.shape)}")
    rows, cols = wp.shape[0], 2 * wp.shape[1]
    groups = cols // 32
    if cols % 32 or tuple(ws.shape) != (rows, groups):
        raise ValueError(
            f"weight_packed {tuple(wp.shape)} encodes [{rows}, {cols}], which needs in % 32 == 0 and "
            f"weight_scale [{rows}, {groups}]; got weight_scale {tuple(ws.shape)}"
        )
    if np.any(ws == 0xFF):
        raise ValueError("E8M0 scale 0xFF is NaN; refusing to load")
    codes = unpack_fp4(wp.reshape(-1), rows * cols).reshape(rows, cols)
    vals = e2m1_decode(codes).astype(np.float64)
    scale = np.ldexp(1.0, ws.astype(np.int64) - 127)
    return (vals.reshape(rows, groups, 32) * scale[..., None]).reshape(rows, cols)
