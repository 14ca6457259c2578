"""Pins the ceil-scale NVFP4 oracle (oracle/nvfp4_ceil_ref.py, the b_r6 rung's convention) on the CPU:
the reference test's named values (tie table, UE4M3 codes, ceil-scale theorem, tightness, nibble
order: tests/kernels/gemm/test_k1_b_r6.py:433-611, in tests/golden/known_answers.json), its laws
(round-trip bound, idempotence, zero blocks, refusal of non-finite operands), and two independent
routes: the UE4M3 ceiling against torch's float8_e4m3fn cast (the same grid, round to nearest even),
and the E2M1 rounding against a brute-force nearest search with an explicit even-index tie rule."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import nvfp4_ceil_ref as C


def test_ue4m3_named_codes(known_answers):
    ka = known_answers["nvfp4_ceil"]["ue4m3_named"]
    assert C.ue4m3_value(ka["codes"]).tolist() == ka["values"]
    assert np.isnan(C.ue4m3_value(ka["nan_code"]))
    assert C.UE4M3_MIN_NORMAL == ka["min_normal"] == C.ue4m3_value(8)


def test_ue4m3_grid_is_torch_e4m3fn():
    """Every finite code decodes to the value torch gives the same E4M3 byte (sign bit clear)."""
    codes = torch.arange(0x7F, dtype=torch.uint8)
    want = codes.view(torch.float8_e4m3fn).to(torch.float64).numpy()
    assert np.array_equal(C.ue4m3_value(codes.numpy()), want)


def test_rne_tie_table(known_answers):
    ka = known_answers["nvfp4_ceil"]["rne_ties"]
    for v, want in zip(ka["in"], ka["out"]):
        assert C.e2m1_value(C.e2m1_round_code(v)) == want, v
        assert C.e2m1_value(C.e2m1_round_code(-v)) == -want, -v
    with pytest.raises(ValueError, match="NanInfEncoding"):
        C.e2m1_round_code(np.inf)


def test_e2m1_sign_rules_code_bytes(known_answers):
    """The two sign rules, compared as code bytes (decoded values cannot tell 0x8 from 0x0): the
    scalar helper sets the sign for every negative input (nvfp4_layout.py:402), the quantizer only
    for a non-zero magnitude (b_r6.py:217-223), which a quantized block shows as well."""
    ka = known_answers["nvfp4_ceil"]
    sc = ka["e2m1_scalar_codes"]
    assert C.e2m1_round_code(np.array(sc["in"])).tolist() == sc["out"]
    for v, want in zip(sc["in"], sc["out"]):
        assert int(C.e2m1_round_code(v)) == want, v
    qc = ka["e2m1_quantizer_codes"]
    assert C._e2m1_quant_code(np.array(qc["in"])).tolist() == qc["out"]
    # a block whose amax is 6 has scale 1 (code 0x38), so y = x and the codes are the quantizer's
    vals = [v for v in qc["in"] if abs(v) > 1e-30 or v == 0.0]
    row = np.zeros(16, np.float32)
    row[0] = 6.0
    row[1:1 + len(vals)] = vals
    packed, scales = C.quantize(row[None, :])
    codes = np.stack((packed & 0xF, packed >> 4), axis=-1).reshape(-1)
    want = [7] + [qc["out"][qc["in"].index(v)] for v in vals] + [0] * (15 - len(vals))
    assert int(scales[0, 0]) == 0x38 and codes.tolist() == want


def test_e2m1_rounding_brute_force():
    """Every midpoint, its float64 neighbours, the grid, a dense sweep and negatives: the nearest
    magnitude by exact float64 distance, ties to the even index (the sign bits are pinned by the
    code-byte known answers above)."""
    mags = np.array(C.E2M1_MAGNITUDES)
    pts = [np.linspace(0, 8, 20001)]
    for m in list(C._MIDS) + list(mags):
        pts.append(np.array([np.nextafter(m, -1), m, np.nextafter(m, 10)]))
    a = np.concatenate(pts)
    a = np.concatenate([a, -a])
    d = np.abs(np.abs(a)[:, None] - mags[None, :])
    best = d.min(axis=1, keepdims=True)
    cand = d == best
    # among tied candidates the even index (mantissa 0) wins
    idx = np.where(cand.sum(1) > 1, np.argmax(cand & (np.arange(8) % 2 == 0), axis=1), np.argmax(cand, axis=1))
    assert np.array_equal(C.e2m1_round_code(a) & 7, idx.astype(np.uint8))
    assert np.array_equal(C._e2m1_quant_code(a) & 7, idx.astype(np.uint8))
    # past the grid it saturates (float64 distances to every anchor tie there, so not brute force)
    assert C.e2m1_round_code([7.0, 1e300, -1e300]).tolist() == [7, 7, 15]


def test_ceil_scale_theorem(known_answers):
    ka = known_answers["nvfp4_ceil"]
    assert int(C.ue4m3_ceil_code(1.0)) == ka["ceil_code_of_1"]
    for amax in ka["ceil_amaxes"]:
        code, scale = C.scale_for_amax(amax)
        assert scale >= amax / C.E2M1_MAX
        assert C.ue4m3_value(code) == scale
        assert amax / scale <= C.E2M1_MAX + 1e-12
    code, scale = C.scale_for_amax(0.0)
    assert int(code) == 0 and float(scale) == 0.0
    with pytest.raises(ValueError, match="exceeds"):
        C.scale_for_amax(C.UE4M3_MAX * C.E2M1_MAX * 2)
    for amax in ka["tight_amaxes"]:
        _, scale = C.scale_for_amax(amax)
        assert scale >= C.UE4M3_MIN_NORMAL
        assert amax / scale >= C.E2M1_MAX / (1 + C.UE4M3_CEIL_RELATIVE) - 1e-12
        assert C.e2m1_value(C.e2m1_round_code(amax / scale)) == C.E2M1_MAX


def test_ceil_against_torch_e4m3_cast():
    """ceil(v) = the round-to-nearest-even E4M3 value when that is >= v, else the next code up."""
    rng = np.random.default_rng(0)
    v = np.concatenate([rng.uniform(0, 448, 4000), np.exp2(rng.uniform(-14, 8.8, 4000)), C._GRID[1:],
                        np.nextafter(C._GRID[1:], 0), np.nextafter(C._GRID[1:-1], 1000), [0.0, 1e-300]])
    v = v[v <= 448]
    r = torch.from_numpy(v).to(torch.float8_e4m3fn)
    rc = r.view(torch.uint8).numpy().astype(np.int64)
    rv = r.to(torch.float64).numpy()
    want = np.where(rv >= v, rc, rc + 1)
    assert np.array_equal(C.ue4m3_ceil_code(v).astype(np.int64), want)


def _scales(x):
    rows, k = x.shape
    amax = np.abs(x.astype(np.float64)).reshape(rows, k // 16, 16).max(-1)
    return C.scale_for_amax(amax)[1]


@pytest.mark.parametrize("magnitude", [1e-3, 1e-2, 1.0, 1e2, 200.0])
def test_round_trip_bound(magnitude):
    """|x - dequant(quant(x))| <= 0.25 * max(|x|, scale) elementwise (test_k1_b_r6.py:517-541)."""
    x = (np.random.default_rng(0).standard_normal((128, 64)) * magnitude).astype(np.float32)
    dq = C.dequantize(*C.quantize(x)).astype(np.float64).reshape(128, 4, 16)
    xb = x.astype(np.float64).reshape(128, 4, 16)
    sc = _scales(x)[..., None]
    assert np.all(np.abs(xb - dq) <= C.E2M1_UNIT_ROUNDOFF * np.maximum(np.abs(xb), sc))
    assert np.abs(xb / np.where(sc > 0, sc, 1)).max() <= C.E2M1_MAX


@pytest.mark.parametrize("magnitude", [1e-1, 1.0, 10.0, 1e2])
def test_idempotent(magnitude):
    x = (np.random.default_rng(1).standard_normal((128, 64)) * magnitude).astype(np.float32)
    assert np.all(_scales(x)[_scales(x) > 0] >= C.UE4M3_MIN_NORMAL)
    p1, s1 = C.quantize(x)
    p2, s2 = C.quantize(C.dequantize(p1, s1))
    assert np.array_equal(p1, p2) and np.array_equal(s1, s2)


def test_zero_blocks_nonfinite_and_nibbles(known_answers):
    x = np.zeros((128, 64), np.float32)
    x[0, :16] = 1.0
    dq = C.dequantize(*C.quantize(x))
    assert np.isfinite(dq).all() and not dq[1:].any()
    for bad in (np.nan, np.inf):
        y = np.zeros((64, 64), np.float32)
        y[3, 7] = bad
        with pytest.raises(ValueError, match="NaN or Inf"):
            C.quantize(y)
    ka = known_answers["nvfp4_ceil"]["nibble_order"]
    z = np.zeros((128, 64), np.float32)
    z[0, 0], z[0, 1] = ka["x0"], ka["x1"]
    p, s = C.quantize(z)
    assert p[0, 0] & 0xF == ka["low_nibble"] and p[0, 0] >> 4 == ka["high_nibble"]
    assert C.dequantize(p, s)[0, :2].tolist() == [ka["x0"], ka["x1"]]
    # negative values that round to zero are stored as +0 (code 0)
    w = np.zeros((1, 16), np.float32)
    w[0, 0], w[0, 1] = 6.0, -0.2
    assert C.quantize(w)[0][0, 0] >> 4 == 0


def test_scales_row_major_and_gemm_is_dequant_product():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((64, 128)).astype(np.float32)
    _, s = C.quantize(x)
    assert np.array_equal(C.ue4m3_value(s), _scales(x))
    a, b = rng.standard_normal((16, 64)).astype(np.float32), rng.standard_normal((64, 24)).astype(np.float32)
    qa = C.dequantize(*C.quantize(a)).astype(np.float64)
    qb = C.dequantize(*C.quantize(b.T.copy())).astype(np.float64)
    assert np.array_equal(C.reference_gemm(a, b), qa @ qb.T)
