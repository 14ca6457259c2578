"""Pins the INT4 oracle (oracle/quant_ref.py) against the reference's known answers, its recorded
SQNR numbers on the reference tests' own seeded data, and closed forms. CPU only."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import quant_ref as R


def test_pack_known_answers(known_answers):
    ka = known_answers["int4_pack"]
    assert R.pack_int4(np.array(ka["high_low_nibble"]["q"], np.int8)).tolist() == ka["high_low_nibble"]["packed"]
    alt = ka["alternating"]
    p = R.pack_int4(np.array(alt["q_pattern"] * alt["repeat"], np.int8))
    assert p.tolist() == [alt["packed_byte"]] * alt["n_bytes"]
    m1 = ka["all_minus_one"]
    p = R.pack_int4(np.full(m1["n"], m1["q_value"], np.int8))
    assert p.tolist() == [m1["packed_byte"]] * m1["n_bytes"]
    odd = np.array(ka["odd_length"]["q"], np.int8)
    p = R.pack_int4(odd)
    assert p.size == ka["odd_length"]["n_bytes"]
    assert R.unpack_int4(p, odd.size).tolist() == odd.tolist()


def test_pack_unpack_full_grid_and_fuzz():
    grid = np.arange(-8, 8, dtype=np.int8)
    assert np.array_equal(R.unpack_int4(R.pack_int4(grid), grid.size), grid)
    rng = np.random.default_rng(0)
    for _ in range(200):
        n = int(rng.integers(1, 300))
        q = rng.integers(-8, 8, n).astype(np.int8)
        assert np.array_equal(R.unpack_int4(R.pack_int4(q), n), q)


def test_unpack_sign_extension_every_byte():
    b = np.arange(256, dtype=np.uint8)
    out = R.unpack_int4(b, 512).astype(int)
    hi, lo = out[0::2], out[1::2]
    for v in range(256):
        h, l = v >> 4, v & 15
        assert hi[v] == (h - 16 if h >= 8 else h) and lo[v] == (l - 16 if l >= 8 else l)


def test_pack_rejects_non_1d():
    with pytest.raises(ValueError, match="1-D"):
        R.pack_int4(np.zeros((2, 2), np.int8))


def test_quantize_rounds_half_to_even():
    # absmax 7 -> scale exactly 1, so w/s is w and every .5 is a true tie (torch.round: half to even).
    w = np.zeros((1, 128), np.float32)
    w[0, :9] = [7.0, 2.5, -2.5, 3.5, 0.5, -0.5, 1.5, 6.5, -6.5]
    q, s = R.quantize_groupwise_int4(w)
    assert s[0, 0] == 1.0
    assert q[0, :9].tolist() == [7, 2, -2, 4, 0, 0, 2, 6, -6]


def test_quantize_scale_is_ieee_division_and_clamped():
    rng = np.random.default_rng(1)
    w = rng.standard_normal((8, 256)).astype(np.float32)
    w[3, 128:] = 0.0  # all-zero group -> FLT_MIN scale, zero codes
    q, s = R.quantize_groupwise_int4(w)
    amax = np.abs(w.reshape(8, 2, 128)).max(-1).astype(np.float64)
    want = (amax / 7.0).astype(np.float32)  # correctly rounded fp32 quotient
    want[3, 1] = np.finfo(np.float32).tiny
    assert np.array_equal(s, want)
    assert np.all(q[3, 128:] == 0)
    # codes never reach -8: |w/s| <= 7 by construction
    assert q.min() >= -7 and q.max() <= 7


def test_quantize_errors():
    with pytest.raises(ValueError, match="2-D"):
        R.quantize_groupwise_int4(np.zeros(128, np.float32))
    with pytest.raises(ValueError, match="not divisible by group_size"):
        R.quantize_groupwise_int4(np.zeros((2, 100), np.float32))


def test_recorded_sqnr_and_granular_floor(known_answers):
    ka = known_answers["int4_sqnr"]
    torch.manual_seed(ka["seed"])
    w = torch.randn(*ka["shape"]).numpy()
    q, s = R.quantize_groupwise_int4(w, ka["group"])
    db = R.sqnr_db(w, R.dequantize_groupwise_int4(q, s, ka["group"]))
    rows, cols = ka["shape"]
    g = cols // ka["group"]
    step = s.reshape(rows, g, 1).astype(np.float64)
    pred = 10 * math.log10((w.astype(np.float64) ** 2).sum() / np.broadcast_to(step**2 / 12, (rows, g, ka["group"])).sum())
    assert abs(db - ka["measured_db"]) < ka["tolerance_db"], db
    assert abs(pred - ka["analytic_db"]) < ka["tolerance_db"], pred


def test_group_beats_per_tensor_recorded():
    # tests/test_quant_int4_group.py:135-149 data; bench/RESULTS.md:560 records 18.69 > 17.12 dB
    torch.manual_seed(3)
    w = torch.randn(64, 128 * 6)
    w[:, 128 * 3 :] *= 20.0
    w = w.numpy()
    qg, sg = R.quantize_groupwise_int4(w)
    qt, st = R.quantize_groupwise_int4(w, group_size=w.shape[1])
    dg = R.sqnr_db(w, R.dequantize_groupwise_int4(qg, sg))
    dt = R.sqnr_db(w, R.dequantize_groupwise_int4(qt, st, w.shape[1]))
    assert abs(dg - 18.69) < 0.01 and abs(dt - 17.12) < 0.01


def test_dequantize_is_correctly_rounded_product():
    rng = np.random.default_rng(2)
    q = rng.integers(-8, 8, (4, 256)).astype(np.int8)
    s = rng.random((4, 2)).astype(np.float32) + np.float32(0.01)
    got = R.dequantize_groupwise_int4(q, s)
    want = (q.astype(np.float64).reshape(4, 2, 128) * s.astype(np.float64)[..., None]).astype(np.float32)
    assert np.array_equal(got, want.reshape(4, 256))


def test_w4a16_linear_law_and_bias():
    # tests/test_quant_int4_group.py:152-182: rel output MSE < 2e-2 vs the fp16 weight, fp16 x
    torch.manual_seed(4)
    w = (torch.randn(512, 1024) * 0.02).numpy()
    x = torch.randn(32, 1024, dtype=torch.float16).float().numpy()
    q, s = R.quantize_groupwise_int4(w)
    y = R.w4a16_linear(x, q, s, act="f16")
    y_ref = R.linear_f64(x, R.round_to(w, "f16"))
    rel = R.mse(y_ref, y) / R.mse(y_ref, np.zeros_like(y_ref))
    assert rel < 2e-2
    bias = np.linspace(-1, 1, 512).astype(np.float32)
    assert np.allclose(R.w4a16_linear(x, q, s, bias=bias, act="f16") - bias, y, atol=1e-9)


def test_w4a16_linear_matches_brute_force():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((5, 64)) * 0.02).astype(np.float32)
    x = R.round_bf16(rng.standard_normal((3, 64)).astype(np.float32))
    q, s = R.quantize_groupwise_int4(w, 32)
    y = R.w4a16_linear(x, q, s, group_size=32)
    for m in range(3):
        for n in range(5):
            acc = 0.0
            for k in range(64):
                wv = float(R.round_bf16(np.float32(float(q[n, k]) * float(s[n, k // 32]))))
                acc += float(x[m, k]) * wv
            assert math.isclose(acc, y[m, n], rel_tol=1e-12, abs_tol=1e-15)


def test_asym_uint4_roundtrip_properties():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((16, 256)) * 0.02).astype(np.float32)
    w[0, :128] = np.abs(w[0, :128])  # one all-positive group: range widened to include 0
    w[1, 5] = 0.0
    q, s, z = R.quantize_groupwise_uint4_asym(w)
    assert q.min() >= 0 and q.max() <= 15
    assert np.all(z == np.rint(z)) and z.min() >= 0 and z.max() <= 15
    assert np.array_equal(s, R.round_bf16(s))  # stored in bf16 without loss
    wd = R.dequantize_groupwise_uint4_asym(q, s, z)
    step = np.repeat(s, 128, axis=1)
    assert np.all(np.abs(wd - w) <= step * 0.5 + 1e-7)
    assert wd[1, 5] == 0.0 or abs(w[1, 5] - wd[1, 5]) <= step[1, 5] / 2
    # true zeros reconstruct exactly because z is an integer code (int8.py:142-172 invariant)
    zero_mask = w == 0.0
    assert np.all(wd[zero_mask] == 0.0)


def test_uint4_asym_invariants():
    """The build-defined asymmetric format has no reference symbol; its oracle is pinned by the
    invariants of an affine quantizer (int8.py:142-172 at 4 bits): real zero reconstructs exactly,
    codes stay in [0, 15], the zero-point is an integer in [0, 15], and every value reconstructs within
    one step s: half a step of rounding, plus up to half a step where the rounded zero-point shifts
    the grid and the top of the range clips (and the bf16 scale may sit 2**-9 below (hi - lo)/15)."""
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((64, 512)) * 0.05 + 0.01).astype(np.float32)
    w[0, :128] = np.abs(w[0, :128])
    w[1, :128] = 0.0
    w[2, 5] = 0.0
    for param in ("f32", "bf16"):
        q, s, z = R.quantize_groupwise_uint4_asym(w, 128, param=param)
        d = R.dequantize_groupwise_uint4_asym(q, s, z)
        assert q.min() >= 0 and q.max() <= 15
        assert np.all(z == np.rint(z)) and z.min() >= 0 and z.max() <= 15 and not np.signbit(z).any()
        assert np.all(d[w == 0] == 0)
        step = np.repeat(s, 128, axis=1)
        assert np.all(np.abs(d - w) <= step * (1 + 2.0**-7))
        inner = (w > -6 * step) & (w < 6 * step)  # well inside the range: rounding error only
        assert np.all(np.abs(d - w)[inner] <= step[inner] / 2 * (1 + 1e-6))
