"""Pins the FP4 oracle (oracle/quant_ref.py: E2M1, E4M3, E8M0, NVFP4, MXFP4, on-disk MXFP4) against
the reference's known answers, its recorded SQNR figures on the reference tests' own seeded data,
golden vectors written by the reference itself (tests/golden/reference_vectors.json), closed forms
and library routines. CPU only."""

from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import quant_ref as R

GOLDEN = Path(__file__).resolve().parent / "golden" / "reference_vectors.json"


@pytest.fixture(scope="module")
def ref_vectors() -> dict:
    return json.loads(GOLDEN.read_text())


def f32(hexes) -> np.ndarray:
    return np.array([struct.unpack("<f", bytes.fromhex(h))[0] for h in hexes], np.float32)


def bits(a) -> np.ndarray:
    return np.asarray(a, np.float32).view(np.uint32)


# ------------------------------------------------------------------------------------ E2M1 codec
def test_e2m1_known_answers(known_answers):
    ka = known_answers["e2m1"]
    grid = np.array(ka["grid"] + [-g for g in ka["grid"]], np.float32)
    assert np.array_equal(np.abs(R.e2m1_decode(R.e2m1_round_to_code(grid))), np.abs(grid))
    near = R.e2m1_decode(R.e2m1_round_to_code(np.array(ka["nearest_in"], np.float32)))
    assert near.tolist() == ka["nearest_out"]
    sat = R.e2m1_decode(R.e2m1_round_to_code(np.array(ka["saturate_in"], np.float32)))
    assert np.all(np.abs(sat) == ka["saturate_abs_out"])


def test_e2m1_golden_specials(ref_vectors):
    """Ties at midpoints go to the lower magnitude; -0 keeps no sign bit but -tiny keeps it;
    inputs whose fp32 distances to every anchor tie (1e30, inf) and NaN give magnitude index 0."""
    g = ref_vectors["e2m1_specials"]
    x = f32(g["x"])
    assert R.e2m1_round_to_code(x).tolist() == g["codes"]


def test_e2m1_midpoints_every_anchor_pair():
    """Brute force: every fp32 input in a window around each midpoint picks the nearer anchor, the
    lower one on an exact tie (the first index of argmin)."""
    mags = np.array(R.FP4_MAGNITUDES, np.float32)
    for lo, hi in zip(mags[:-1], mags[1:]):
        mid = np.float32((lo + hi) / 2)
        u = mid.view(np.uint32)
        window = (np.arange(-64, 65, dtype=np.int64) + int(u)).astype(np.uint32).view(np.float32)
        codes = R.e2m1_round_to_code(window)
        want = np.where(window <= mid, np.searchsorted(mags, lo), np.searchsorted(mags, hi))
        assert np.array_equal(codes & 7, want.astype(np.uint8)), (lo, hi)


def test_e2m1_decode_named_bytes(known_answers):
    ka = known_answers["mxfp4_checkpoint_named"]
    codes = R.unpack_fp4(np.array(ka["bytes"], np.uint8), 6)
    assert R.e2m1_decode(codes).tolist() == ka["scale_127_values"]
    assert np.signbit(R.e2m1_decode(codes))[1]  # 0x80 high nibble decodes to -0.0


def test_fp4_pack_unpack_roundtrip():
    rng = np.random.default_rng(0)
    for n in (1, 2, 3, 17, 4096, 4097):
        c = rng.integers(0, 16, n).astype(np.uint8)
        p = R.pack_fp4(c)
        assert p.size == (n + 1) // 2
        assert np.array_equal(R.unpack_fp4(p, n), c)
    assert R.pack_fp4(np.array([1, 2], np.uint8)).tolist() == [0x21]  # even element in the low nibble


# ------------------------------------------------------------------------------------ scale codecs
def test_e4m3_known_answers(known_answers):
    ka = known_answers["e4m3"]
    v = np.array(ka["self_map"], np.float32)
    assert np.array_equal(R.quantize_e4m3(v), v)
    assert R.quantize_e4m3(np.array([ka["saturate_in"]], np.float32))[0] == ka["saturate_out"]


def test_e4m3_matches_library_rne_over_range():
    """The E4M3 grid with round-half-even is torch's float8_e4m3fn cast for finite in-range values."""
    u = np.arange(0x00000001, 0x43E00000, 4099, dtype=np.uint64).astype(np.uint32)
    v = u.view(np.float32)
    v = v[(v > 0) & (v <= 448.0)]
    lib = torch.from_numpy(v.copy()).to(torch.float8_e4m3fn).to(torch.float32).numpy()
    assert np.array_equal(R.quantize_e4m3(v), lib)


def test_e4m3_golden_edges(ref_vectors):
    g = ref_vectors["e4m3_edges"]
    assert np.array_equal(bits(R.quantize_e4m3(f32(g["v"]))), bits(f32(g["out"])))


def test_e8m0_known_answers_and_golden(known_answers, ref_vectors):
    v = np.array(known_answers["e8m0"]["self_map"], np.float32)
    assert np.array_equal(R.quantize_e8m0(v), v)
    g = ref_vectors["e8m0_midpoints"]
    assert np.array_equal(bits(R.quantize_e8m0(f32(g["v"]))), bits(f32(g["out"])))


def test_mxfp4_scale_at_powers_of_two_golden(ref_vectors):
    """911 blocks whose amax/6 sits at or a few ulps either side of a power of two: the reference's
    scale is the ceil of the fp32 log2, which differs from the exact ceil on 241 of them."""
    g = ref_vectors["mxfp4_scale_edges"]
    rows = g["rows"]
    x = np.zeros((rows, 32), np.float32)
    x[:, :5] = f32(g["x_head"]).reshape(rows, 5)
    codes, s_block, e8, _, _ = R.mxfp4_quantize(x, 32)
    assert np.array_equal(bits(s_block), bits(f32(g["s_block"])))
    assert codes[:, :5].reshape(-1).tolist() == g["codes_head"]
    assert g["tail_codes_zero"] and np.all(codes[:, 5:] == 0)
    assert np.array_equal(np.ldexp(np.float32(1), e8.astype(np.int32) - 127), s_block)


# ------------------------------------------------------------------------------------ NVFP4 / MXFP4
def test_small_tensors_golden(ref_vectors):
    g = ref_vectors["nvfp4_small"]
    x = f32(g["x"]).reshape(g["shape"])
    codes, s_global, s_block, _, _ = R.nvfp4_quantize(x, 16)
    assert codes.reshape(-1).tolist() == g["codes"]
    assert np.array_equal(bits(s_block), bits(f32(g["s_block"])))
    assert bits(np.float32(s_global)) == bits(f32([g["s_global"]]))[0]
    g = ref_vectors["mxfp4_small"]
    x = f32(g["x"]).reshape(g["shape"])
    codes, s_block, _, _, _ = R.mxfp4_quantize(x, 32)
    assert codes.reshape(-1).tolist() == g["codes"]
    assert np.array_equal(bits(s_block), bits(f32(g["s_block"])))


def test_recorded_sqnr_nvfp4_vs_mxfp4(known_answers):
    """bench/RESULTS.md:561 on the reference test's data (torch.manual_seed(0); randn(8192, 256))."""
    ka = known_answers["nvfp4_vs_mxfp4"]
    torch.manual_seed(ka["seed"])
    x = torch.randn(*ka["shape"]).numpy()
    nv = R.nvfp4_dequantize(*R.nvfp4_quantize(x, 16))
    c, s, _, shp, n = R.mxfp4_quantize(x, 32)
    mx = R.mxfp4_dequantize(c, s, shp, n)
    assert abs(R.sqnr_db(x, nv) - ka["nvfp4_db"]) < ka["tolerance_db"]
    assert abs(R.sqnr_db(x, mx) - ka["mxfp4_db"]) < ka["tolerance_db"]
    assert abs(R.mse(x, mx) / R.mse(x, nv) - ka["mse_ratio"]) < 0.01


def test_nvfp4_linear_block_accumulation_law():
    """quant_linear_nvfp4 == x @ nvfp4_dequant(W).T to < 1e-4 (tests/test_quant_nvfp4_mxfp4.py:183-193)."""
    torch.manual_seed(4)
    x = torch.randn(64, 512).numpy()
    w = torch.randn(256, 512).numpy()
    y = R.quant_linear_nvfp4(x, w, 16)
    w_hat = R.nvfp4_dequantize(*R.nvfp4_quantize(w, 16))
    y_ref = x.astype(np.float64) @ w_hat.astype(np.float64).T
    assert np.linalg.norm(y - y_ref) / np.linalg.norm(y_ref) < 1e-4
    with pytest.raises(ValueError, match="multiple of block"):
        R.quant_linear_nvfp4(np.zeros((4, 30), np.float32), np.zeros((8, 30), np.float32), 16)


# ------------------------------------------------------------------------------------ on-disk MXFP4
def test_checkpoint_decode_every_byte_every_scale():
    """k3/checkpoint.py:92-144 against an independent bit-level decoder over all 256 bytes x all 255
    finite scale codes (tests/test_k3_checkpoint.py:260-278)."""
    packed = np.repeat(np.arange(256, dtype=np.uint8)[None, :], 255, axis=0)  # [255, 256] -> in 512
    packed = packed.reshape(255 * 16, 16)  # rows of 32 codes, one scale per row
    scale = np.repeat(np.arange(255, dtype=np.uint8), 16).reshape(255 * 16, 1)
    w = R.dequantize_mxfp4_checkpoint(packed, scale)

    def bit_decode(nib: int) -> float:
        s = -1.0 if nib & 8 else 1.0
        e, m = (nib >> 1) & 3, nib & 1
        return s * (m * 0.5 if e == 0 else 2.0 ** (e - 1) * (1 + m * 0.5))

    table = np.array([bit_decode(n) for n in range(16)])
    lo, hi = table[packed & 0xF], table[packed >> 4]
    want = np.stack([lo, hi], axis=-1).reshape(packed.shape[0], 32) * np.ldexp(1.0, scale.astype(np.int64) - 127)
    assert np.array_equal(w, want)
    with pytest.raises(ValueError, match="NaN"):
        R.dequantize_mxfp4_checkpoint(np.zeros((1, 16), np.uint8), np.full((1, 1), 255, np.uint8))
