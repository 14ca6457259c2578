"""Pins the FP8 oracle (oracle/fp8_ref.py) on the CPU: torch's own float8_e4m3fn casts, the
reference's named values and laws (tests/quant/test_s1_s_r2.py), brute force."""

from __future__ import annotations

import numpy as np
import torch

from oracle import fp8_ref as F

FP8 = torch.float8_e4m3fn


def _torch_sat(v: np.ndarray) -> np.ndarray:
    return torch.from_numpy(v).clamp(-448.0, 448.0).to(FP8).view(torch.uint8).numpy()


def _grid() -> np.ndarray:
    vals = np.array([F.e4m3_decode(c) for c in range(127)], dtype=np.float64).ravel()
    mids = (vals[:-1] + vals[1:]) / 2
    pts = np.concatenate([vals, mids]).astype(np.float32)
    nb = np.concatenate([np.nextafter(pts, np.float32(np.inf)), np.nextafter(pts, np.float32(-np.inf))])
    dense = np.logspace(-12, 20, 20001, base=2.0).astype(np.float32)
    special = np.array([0.0, 448.0, 449.0, 463.9, 464.0, 464.1, 480.0, 1e5, 3e38, np.inf, 2.0**-10,
                        2.0**-10 * 1.0000001, 2.0**-11, 1e-30, 1e-45], dtype=np.float32)
    g = np.concatenate([pts, nb, dense, special]).astype(np.float32)
    return np.concatenate([g, -g])


def test_encode_matches_torch_cast_everywhere():
    v = _grid()
    got = F.e4m3_encode_sat(v)
    want = _torch_sat(v)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} differ, first {v[bad[:5]]}: {got[bad[:5]]} vs {want[bad[:5]]}"
    # NaN keeps its sign and becomes the NaN code, as torch's cast does
    nan = np.array([np.nan, -np.nan], dtype=np.float32)
    assert np.array_equal(F.e4m3_encode_sat(nan) & 0x7F, np.array([0x7F, 0x7F], dtype=np.uint8))
    assert np.array_equal(F.e4m3_encode_sat(nan) & 0x7F, _torch_sat(nan) & 0x7F)


def test_decode_matches_torch_for_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(FP8).float().numpy()
    got = F.e4m3_decode(codes)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))


def test_named_values_of_the_raw_cast_and_the_clamp():
    """tests/quant/test_s1_s_r2.py:203-223: the raw cast saturates on [448, 464] and is NaN above."""
    raw = torch.tensor([448.0, 464.0, 465.0, 1e5]).to(FP8).float()
    assert raw[0] == 448 and raw[1] == 448 and torch.isnan(raw[2]) and torch.isnan(raw[3])
    clamped = F.e4m3_decode(F.e4m3_encode_sat(np.array([448.0, 464.0, 465.0, 1e5], dtype=np.float32)))
    assert clamped.tolist() == [448.0, 448.0, 448.0, 448.0]


def test_quantize_rows_laws():
    """tests/quant/test_s1_s_r2.py:134-200: round trip within E4M3's own quantum, each row reaching
    448, per-row independence."""
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((32, 128)) * np.logspace(-3, 3, 32)[:, None]).astype(np.float32)
    codes, scale = F.quantize_rows(w)
    assert scale.shape == (32, 1)
    v = (w / scale).astype(np.float32)
    q = F.e4m3_decode(codes)
    err = np.abs(v - q)
    normal = np.abs(v) >= 2.0**-6
    assert np.all(err[normal] <= 2.0**-4 * np.abs(v[normal]))
    assert np.all(err[~normal] <= 2.0**-10)
    assert np.all(np.abs(q).max(axis=1) == 448.0)
    # the scale is the reference's torch expression
    ts = (torch.from_numpy(w).abs().amax(dim=1, keepdim=True) / 448.0).clamp_min(1.0 / (448.0 * 512.0))
    assert np.array_equal(scale.view(np.uint32), ts.numpy().view(np.uint32))
    x2 = w.copy()
    x2[0] *= 1000.0
    c2, _ = F.quantize_rows(x2)
    assert np.array_equal(c2[1:], codes[1:])
    # an all-zero row takes the MIN_SCALE floor and zero codes
    cz, sz = F.quantize_rows(np.zeros((1, 16), dtype=np.float32))
    assert sz[0, 0] == np.float32(1.0 / (448.0 * 512.0)) and not cz.any()


def test_per_head_flush_idempotence_and_saturation():
    """tests/quant/test_s1_s_r2.py:278-348."""
    x = np.zeros((1, 1, 4, 2), dtype=np.float32)
    x[0, 0, 0, 0] = 1.0
    s = F.per_head_scale(x)
    unit = float(s[0, 0, 0, 0])
    x[0, 0, 1, 0] = unit * (2.0**-9 / 2) * 0.9
    x[0, 0, 2, 0] = unit * 2.0**-9
    out = F.dequantize_per_head(F.quantize_per_head(x, s), s)
    assert out[0, 0, 1, 0] == 0.0
    assert abs(out[0, 0, 2, 0] - unit * 2.0**-9) <= 1e-6 * unit * 2.0**-9
    rng = np.random.default_rng(3)
    kv = (rng.standard_normal((2, 4, 8, 16)) * np.logspace(-3, 3, 4)[None, :, None, None]).astype(np.float32)
    sc = F.per_head_scale(kv)
    once = F.quantize_per_head(kv, sc)
    twice = F.quantize_per_head(F.dequantize_per_head(once, sc), sc)
    assert np.array_equal(once, twice)
    over = kv.copy()
    over[:, 0] = np.abs(over[:, 0]) * 1e4 + 1.0
    n = F.saturated_count(over, sc)
    assert n > 0
    q = F.dequantize_per_head(F.quantize_per_head(over, sc), sc)
    assert not np.isnan(q).any()


def test_fp8_linear_reference_is_a_matmul():
    """tests/quant/test_s1_s_r2.py:401-416."""
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 4)).astype(np.float32)
    w = rng.standard_normal((5, 4)).astype(np.float32)
    wc, ws = F.quantize_rows(w)
    bias = rng.standard_normal(5)
    got = F.fp8_linear_reference(x, wc, ws, bias)
    xc, xs = F.quantize_rows(x)
    xd = F.e4m3_decode(xc).astype(np.float64) * xs
    wd = F.e4m3_decode(wc).astype(np.float64) * ws
    for m in range(3):
        for n in range(5):
            want = sum(xd[m, k] * wd[n, k] for k in range(4)) + bias[n]
            assert abs(got[m, n] - want) <= 1e-12 * max(1.0, abs(want))
