"""Pins the INT8 oracle (oracle/quant_ref.py) against the reference's known answers, its recorded
SQNR figures on the reference tests' own seeded data, and torch's own bf16 / fp16 arithmetic (the
rounding model the oracle uses for inputs in those dtypes). CPU only."""

from __future__ import annotations

import numpy as np
import torch

from oracle import quant_ref as R


def test_book_example(known_answers):
    ka = known_answers["int8_book"]
    q, s = R.quantize_symmetric(np.array(ka["x"], np.float32))
    assert q.tolist() == ka["codes"]
    assert s == np.float32(2.5) / np.float32(127)
    x_hat = R.dequantize_symmetric(q, s)
    assert x_hat[2] == np.float32(2.5)


def test_recorded_sqnr(known_answers):
    """bench/RESULTS.md:558-559 on the reference tests' data (tests/test_quant_int8.py:38-118)."""
    ka = known_answers["int8_sqnr"]
    tol = ka["tolerance_db"]
    torch.manual_seed(0)
    x = torch.randn(4096).numpy()
    assert abs(R.sqnr_db(x, R.dequantize_symmetric(*R.quantize_symmetric(x))) - ka["sym_gaussian_seed0_n4096_db"]) < tol
    torch.manual_seed(1)
    x = (torch.relu(torch.randn(8192)) ** 1.5).numpy()
    aff = R.dequantize_affine(*R.quantize_affine(x))
    sym = R.dequantize_symmetric(*R.quantize_symmetric(x))
    assert abs(R.sqnr_db(x, aff) - ka["affine_skewed_seed1_db"]) < tol
    assert abs(R.sqnr_db(x, sym) - ka["sym_skewed_seed1_db"]) < tol
    torch.manual_seed(3)
    w = (torch.randn(32, 512) * torch.logspace(-2, 1, 32).unsqueeze(1)).numpy()
    pt = R.dequantize_symmetric(*R.quantize_symmetric(w, axis=None))
    pc = R.dequantize_symmetric(*R.quantize_symmetric(w, axis=0))
    assert abs(R.sqnr_db(w, pt) - ka["per_tensor_seed3_db"]) < tol
    assert abs(R.sqnr_db(w, pc) - ka["per_channel_seed3_db"]) < tol


def test_affine_zero_exact():
    """tests/test_quant_int8.py:89-100: true zeros reconstruct exactly."""
    torch.manual_seed(2)
    x = torch.relu(torch.randn(1000)).numpy()
    x_hat = R.dequantize_affine(*R.quantize_affine(x))
    assert np.all(x_hat[x == 0] == 0)


def test_w8a8_law_and_exact_integer_core():
    torch.manual_seed(4)
    x = torch.randn(64, 256)
    w = torch.randn(128, 256) * torch.logspace(-1, 1, 128).unsqueeze(1)
    y = R.w8a8_linear(x.numpy(), w.numpy())
    y_ref = (x @ w.t()).numpy().astype(np.float64)
    assert np.linalg.norm(y - y_ref) / np.linalg.norm(y_ref) < 1.5e-2
    # the integer core is exact: brute-force int64 sums on a slice
    qx, sx = R.quantize_symmetric(x.numpy(), axis=0)
    qw, sw = R.quantize_symmetric(w.numpy(), axis=0)
    acc = sum(int(qx[3, k]) * int(qw[7, k]) for k in range(256))
    assert y[3, 7] == np.float32(acc) * (sx[3, 0] * sw[7, 0])


def test_dtype_rounding_model_matches_torch():
    """torch's bf16 / fp16 elementwise ops round each fp32 result to the dtype: the oracle's model of
    the reference computing in x's dtype reproduces torch's own bf16 / fp16 arithmetic bit for bit."""
    g = torch.Generator().manual_seed(9)
    x32 = torch.randn(64, 300, generator=g) * 3
    for tdt, name in ((torch.bfloat16, "bf16"), (torch.float16, "f16")):
        x = x32.to(tdt)
        amax = x.abs().amax(dim=1, keepdim=True)
        s = (amax / 127).clamp_min(1e-12)
        q = torch.round(x / s).clamp(-127, 127).to(torch.int8)
        qo, so = R.quantize_symmetric(x.float().numpy(), axis=0, dtype=name)
        assert np.array_equal(qo, q.numpy()) and np.array_equal(so, s.float().numpy())
        lo = torch.minimum(x.amin(dim=0, keepdim=True), torch.zeros(1, dtype=tdt))
        hi = torch.maximum(x.amax(dim=0, keepdim=True), torch.zeros(1, dtype=tdt))
        sa = ((hi - lo) / 255).clamp_min(1e-12)
        za = torch.round(-lo / sa).clamp(0, 255)
        qa = torch.round(x / sa + za).clamp(0, 255).to(torch.uint8)
        qo, so, zo = R.quantize_affine(x.float().numpy(), axis=1, dtype=name)
        assert np.array_equal(qo, qa.numpy())
        assert np.array_equal(so, sa.float().numpy()) and np.array_equal(zo, za.float().numpy())
        d = (qa.to(tdt) - za) * sa
        assert np.array_equal(R.dequantize_affine(qo, so, zo, dtype=name), d.float().numpy())
