"""INT8 parity on the MI355X: the HIP kernels (through libsqx_hip.so) against the numpy oracle.

Bit-exact: quantize_symmetric / quantize_affine (codes, scales, zero-points) for fp32, bf16 and fp16
inputs, per-tensor and along every axis; dequantize; w8a8_linear (exact int32 core and the
reference's fp32 epilogue). The weight-only linear is checked within
max|y - y_ref| / max|y_ref| <= 1e-2 of the float64 product of x and (q*s).to(x.dtype), plus the
elementwise bound |y - y_ref| <= 2**-7 (|y_ref| + rms(y_ref)).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import quant_ref as R
from tests.conftest import print_case

pytestmark = pytest.mark.gpu
DEV = "cuda"
DT = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}


@pytest.fixture(scope="module")
def i8():
    from scratch_llm_amd import _lib
    from scratch_llm_amd.quant import int8

    _lib.load()
    return int8


def _data(shape, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * torch.logspace(-2, 1, shape[-1] if len(shape) else 1)
    if x.numel() > 8:
        x.view(-1)[:4] = torch.tensor([0.0, -0.0, 1e-3, -2.5])
    return x.to(dtype)


def bits(a) -> np.ndarray:
    a = np.ascontiguousarray(np.asarray(a, np.float32))
    return a.view(np.uint32)


CASES = [((4096,), None), ((32, 512), None), ((32, 512), 0), ((64, 300), 1), ((64, 300), -1),
         ((4, 6, 70), 1), ((4, 6, 70), 0), ((4, 6, 70), 2), ((300, 4096), 0), ((1 << 20,), None)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape,axis", CASES)
def test_quantize_symmetric_bitexact(i8, shape, axis, dtype):
    print_case("int8 sym", shape, axis, dtype)
    x = _data(shape, len(shape) * 100 + (axis or 0), dtype)
    q, s = i8.quantize_symmetric(x.to(DEV), axis=axis)
    qr, sr = R.quantize_symmetric(x.float().numpy(), axis=axis, dtype=DT[dtype])
    assert q.dtype == torch.int8 and s.dtype == dtype and tuple(s.shape) == tuple(np.shape(sr))
    assert np.array_equal(q.cpu().numpy(), qr)
    assert np.array_equal(bits(s.float().cpu().numpy()), bits(sr))
    d = i8.dequantize_symmetric(q, s)
    assert d.dtype == dtype
    assert np.array_equal(bits(d.float().cpu().numpy()), bits(R.dequantize_symmetric(qr, sr, DT[dtype])))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape,axis", CASES)
def test_quantize_affine_bitexact(i8, shape, axis, dtype):
    print_case("int8 affine", shape, axis, dtype)
    x = _data(shape, len(shape) * 200 + (axis or 0), dtype)
    if x.numel() > 64:
        x.view(-1)[10:40] = x.view(-1)[10:40].abs()  # a positive run
    q, s, z = i8.quantize_affine(x.to(DEV), axis=axis)
    qr, sr, zr = R.quantize_affine(x.float().numpy(), axis=axis, dtype=DT[dtype])
    assert q.dtype == torch.uint8 and s.dtype == dtype and z.dtype == dtype
    assert np.array_equal(q.cpu().numpy(), qr)
    assert np.array_equal(bits(s.float().cpu().numpy()), bits(sr))
    assert np.array_equal(bits(z.float().cpu().numpy()), bits(zr))
    d = i8.dequantize_affine(q, s, z)
    assert np.array_equal(bits(d.float().cpu().numpy()), bits(R.dequantize_affine(qr, sr, zr, DT[dtype])))


def test_book_example_and_zero_exact(i8, known_answers):
    ka = known_answers["int8_book"]
    q, s = i8.quantize_symmetric(torch.tensor(ka["x"], device=DEV))
    assert q.cpu().tolist() == ka["codes"]
    torch.manual_seed(2)
    x = torch.relu(torch.randn(1000)).to(DEV)
    x_hat = i8.fake_quant_affine(x)
    assert torch.all(x_hat[x == 0] == 0)


def test_recorded_sqnr_on_gpu(i8, known_answers):
    ka = known_answers["int8_sqnr"]
    torch.manual_seed(3)
    w = (torch.randn(32, 512) * torch.logspace(-2, 1, 32).unsqueeze(1)).to(DEV)
    assert abs(i8.sqnr_db(w, i8.fake_quant_symmetric(w, axis=None)) - ka["per_tensor_seed3_db"]) < ka["tolerance_db"]
    assert abs(i8.sqnr_db(w, i8.fake_quant_symmetric(w, axis=0)) - ka["per_channel_seed3_db"]) < ka["tolerance_db"]


@pytest.mark.parametrize("m,k,n,dtype", [(64, 256, 128, torch.float32), (5, 300, 33, torch.float32),
                                         (17, 4096, 64, torch.bfloat16), (1, 100, 7, torch.float16),
                                         (128, 1024, 96, torch.float32)])
def test_w8a8_linear_bitexact(i8, m, k, n, dtype):
    print_case("w8a8", m, k, n, dtype)
    g = torch.Generator().manual_seed(m * k + n)
    x = torch.randn(m, k, generator=g).to(dtype)
    w = (torch.randn(n, k, generator=g) * torch.logspace(-1, 1, n).unsqueeze(1)).to(dtype)
    y = i8.w8a8_linear(x.to(DEV), w.to(DEV))
    assert y.dtype == torch.float32 and y.shape == (m, n)
    y_ref = R.w8a8_linear(x.float().numpy(), w.float().numpy(), dtype=DT[dtype])
    assert np.array_equal(bits(y.cpu().numpy()), bits(y_ref))


def test_w8a8_linear_law_and_batch(i8):
    torch.manual_seed(4)
    x = torch.randn(64, 256)
    w = torch.randn(128, 256) * torch.logspace(-1, 1, 128).unsqueeze(1)
    y = i8.w8a8_linear(x.to(DEV), w.to(DEV)).cpu()
    y_ref = x @ w.t()
    assert float((y - y_ref).norm() / y_ref.norm()) < 1.5e-2
    yb = i8.w8a8_linear(x.reshape(8, 8, 256).to(DEV), w.to(DEV)).cpu()
    assert yb.shape == (8, 8, 128) and torch.equal(yb.reshape(64, 128), y)


def _check_linear(y_gpu, y_ref, what):
    y = y_gpu.float().cpu().numpy().astype(np.float64)
    err = np.abs(y - y_ref)
    rel = float(err.max() / np.abs(y_ref).max())
    rms = float(np.sqrt((y_ref**2).mean()))
    worst = float((err / (2.0**-7 * (np.abs(y_ref) + rms))).max())
    assert rel <= 1e-2, f"{what}: max-abs-rel {rel:.3e}"
    assert worst <= 1.0, f"{what}: elementwise bound exceeded {worst:.2f}x"


@pytest.mark.parametrize("m", [1, 16])
def test_int8_weight_linear_config1(i8, m):
    """W 4096x4096 bf16 ~N(0, 0.02) -> quantize_symmetric(W.float(), axis=0)."""
    print_case("int8 config1", m)
    g = torch.Generator(device=DEV).manual_seed(1001)
    w = (torch.randn(4096, 4096, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    q, s = i8.quantize_symmetric(w.float(), axis=0)
    qr, sr = R.quantize_symmetric(w.float().cpu().numpy(), axis=0)
    assert np.array_equal(q.cpu().numpy(), qr) and np.array_equal(bits(s.cpu().numpy()), bits(sr))
    x = torch.randn(m, 4096, generator=g, device=DEV).to(torch.bfloat16)
    y = i8.int8_weight_linear(x, q, s)
    w_eff = R.round_bf16(R.dequantize_symmetric(qr, sr))
    _check_linear(y, R.linear_f64(x.float().cpu().numpy(), w_eff), f"int8 config1 M={m}")


@pytest.mark.parametrize("n,k,m,dtype", [(1000, 1024, 3, torch.bfloat16), (40, 200, 5, torch.float16),
                                         (64, 4096, 64, torch.bfloat16), (16, 64, 100, torch.bfloat16),
                                         # the one-row form: ragged rows, fp16, a K tail, > 1024 tiles
                                         (1000, 1024, 1, torch.bfloat16), (40, 200, 1, torch.float16),
                                         (20000, 256, 1, torch.bfloat16)])
def test_int8_weight_linear_ragged(i8, n, k, m, dtype):
    print_case("int8 ragged", n, k, m, dtype)
    g = torch.Generator(device=DEV).manual_seed(n + k + m)
    w = torch.randn(n, k, generator=g, device=DEV) * 0.05
    q, s = i8.quantize_symmetric(w, axis=0)
    x = torch.randn(m, k, generator=g, device=DEV).to(dtype)
    bias = torch.randn(n, generator=g, device=DEV).to(dtype)
    y = i8.int8_weight_linear(x, q, s, bias)
    act = "bf16" if dtype == torch.bfloat16 else "f16"
    w_eff = R.round_to(R.dequantize_symmetric(q.cpu().numpy(), s.cpu().numpy()), act)
    _check_linear(y, R.linear_f64(x.float().cpu().numpy(), w_eff, bias.float().cpu().numpy()), f"{k}->{n} M={m}")
