"""AWQ and asymmetric uint4 parity on the MI355X: HIP kernels against the numpy oracle.

Bit-exact: quantize_awq_int4 with a channel scale (codes and group scales of W*s), awq_dequantize,
the fake-quantized search weight, the asymmetric uint4 quantizer. act_scale and the grid scale are
within 2e-6 relative (fp64 vs torch's fp32 summation order). search_awq_scale picks the reference's
alpha on the reference test layers (golden vectors). awq_linear at BASELINE config 3 shapes is within
max|y - y_ref| / max|y_ref| <= 1e-2 of the float64 product of x and the bf16-cast effective weight,
and within the elementwise bound |y - y_ref| <= 2**-6 (|y_ref| + rms(y_ref)): twice the bound of the
plain W4A16 linear, because two independent bf16 roundings enter each product here (the kernel's
x/s and the reference's bf16 effective weight) against one there.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import quant_ref as R
from tests.conftest import print_case
from tests.test_oracle_awq import awq_layer

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLDEN = Path(__file__).resolve().parent / "golden" / "reference_vectors.json"


@pytest.fixture(scope="module")
def aw():
    from scratch_llm_amd import _lib
    from scratch_llm_amd.quant import awq

    _lib.load()
    return awq


def bits(a):
    return np.ascontiguousarray(np.asarray(a, np.float32)).view(np.uint32)


def _chan_scale(k, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.exp(torch.empty(k).uniform_(np.log(0.5), np.log(2.0), generator=g))  # log-uniform [0.5, 2]


@pytest.mark.parametrize("n,k,group,dtype", [(256, 512, 128, torch.float32), (4096, 4096, 128, torch.bfloat16),
                                             (96, 384, 64, torch.float32), (40, 96, 32, torch.float16),
                                             (8, 384, 96, torch.float32)])
def test_quantize_awq_with_scale_bitexact(aw, n, k, group, dtype):
    print_case("awq quantize", n, k, group, dtype)
    g = torch.Generator().manual_seed(n + k)
    w = (torch.randn(n, k, generator=g) * 0.02).to(dtype)
    s = _chan_scale(k, n)
    qt = aw.quantize_awq_int4(w.to(DEV), chan_scale=s.to(DEV), group_size=group)
    q, gs, _ = R.quantize_awq_int4(w.float().numpy(), s.numpy(), group)
    assert np.array_equal(qt.q.cpu().numpy(), q)
    assert np.array_equal(bits(qt.group_scales.cpu().numpy()), bits(gs))
    d = aw.awq_dequantize(qt).cpu().numpy()
    assert np.array_equal(bits(d), bits(R.awq_dequantize(q, gs, s.numpy(), group)))
    fake = aw._awq_dequant_weight(w.to(DEV), s.to(DEV), group).cpu().numpy()
    assert np.array_equal(bits(fake), bits(R.awq_dequantize(q, gs, s.numpy(), group)))


def test_act_scale_and_grid_scale(aw):
    w, x, _ = awq_layer(3)
    a = aw.act_scale(torch.from_numpy(x).to(DEV)).cpu().numpy()
    ar = R.act_scale(x)
    assert np.allclose(a, ar, rtol=2e-6, atol=0)
    for ratio in (0.0, 0.25, 0.5, 1.0):
        s = aw._grid_scale(torch.from_numpy(ar).to(DEV), ratio).cpu().numpy()
        sr = R.normalize_scale(np.power(ar, np.float32(ratio)).astype(np.float32))
        assert np.allclose(s, sr, rtol=2e-6, atol=0), ratio


def test_search_picks_reference_alpha(aw):
    cases = json.loads(GOLDEN.read_text())["awq_search"]["cases"]
    for c in cases:
        print_case("awq search", c["seed"])
        w, x, _ = awq_layer(c["seed"])
        res = aw.search_awq_scale(torch.from_numpy(w).to(DEV), torch.from_numpy(x).to(DEV))
        assert res.ratio == c["ratio"]
        assert abs(res.calib_mse - c["calib_mse"]) <= 1e-3 * c["calib_mse"]


def test_awq_laws_on_gpu(aw, known_answers):
    """tests/test_quant_awq.py:61-127 laws, on the GPU path end to end (fp32 x, as the reference)."""
    ka = known_answers["awq"]
    w, x, sal = awq_layer(0)
    wt, xt = torch.from_numpy(w).to(DEV), torch.from_numpy(x).to(DEV)
    y_ref = xt @ wt.t()
    from scratch_llm_amd.quant import int4_group as q4

    qn, sn = q4.quantize_groupwise_int4(wt)
    m_n = q4.mse(y_ref, xt @ q4.dequantize_groupwise_int4(qn, sn).t())
    quant = aw.quantize_awq_int4(wt, x=xt)
    m_a = q4.mse(y_ref, aw.awq_linear(xt, quant))
    assert m_n / m_a > ka["recovery_min"]
    ones = torch.ones(512, device=DEV)
    assert torch.equal(aw.quantize_awq_int4(wt, chan_scale=ones).q, qn)
    res = aw.search_awq_scale(wt, xt)
    assert res.chan_scale[torch.from_numpy(sal).to(DEV)].mean() > res.chan_scale.median()
    assert 0.0 < res.ratio < 1.0
    y_direct = xt @ aw.awq_dequantize(quant).t()
    assert torch.allclose(y_direct, aw.awq_linear(xt, quant), atol=1e-5)


def _check_linear(y_gpu, y_ref, what):
    y = y_gpu.float().cpu().numpy().astype(np.float64)
    err = np.abs(y - y_ref)
    rel = float(err.max() / np.abs(y_ref).max())
    rms = float(np.sqrt((y_ref**2).mean()))
    worst = float((err / (2.0**-6 * (np.abs(y_ref) + rms))).max())
    assert rel <= 1e-2, f"{what}: max-abs-rel {rel:.3e}"
    assert worst <= 1.0, f"{what}: elementwise bound exceeded {worst:.2f}x"


@pytest.mark.parametrize("n,k", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)])
@pytest.mark.parametrize("m", [1, 8, 64, 512])
def test_awq_linear_config3(aw, n, k, m):
    """s ~ log-uniform[0.5, 2] folded into W before quantization; x bf16 ~N(0,1)
    with 1% of channels x20."""
    print_case("awq linear", n, k, m)
    g = torch.Generator(device=DEV).manual_seed(n + k + m)
    w = torch.randn(n, k, generator=g, device=DEV) * 0.02
    s = _chan_scale(k, k).to(DEV)
    quant = aw.quantize_awq_int4(w, chan_scale=s)
    x = torch.randn(m, k, generator=g, device=DEV)
    out_ch = torch.randperm(k, generator=torch.Generator().manual_seed(k))[: k // 100].to(DEV)
    x[:, out_ch] *= 20.0
    x = x.to(torch.bfloat16)
    y = aw.awq_linear(x, quant)
    rows = min(m, 64)  # the float64 reference on a row subset keeps the CPU time bounded
    w_eff = R.round_bf16(aw.awq_dequantize(quant).cpu().numpy())
    _check_linear(y[:rows], R.linear_f64(x[:rows].float().cpu().numpy(), w_eff), f"awq {k}->{n} M={m}")


@pytest.mark.parametrize("group,m", [(256, 1), (512, 8), (4096, 64), (1024, 300)])
def test_awq_linear_wide_groups(aw, group, m):
    """AWQ with groups wider than 128 (awq.py:184-192 takes any group dividing in_features)."""
    print_case("awq wide group", group, m)
    n, k = 512, 4096
    g = torch.Generator(device=DEV).manual_seed(group + m)
    w = torch.randn(n, k, generator=g, device=DEV) * 0.02
    s = _chan_scale(k, group).to(DEV)
    quant = aw.quantize_awq_int4(w, chan_scale=s, group_size=group)
    assert quant.group_scales.shape == (n, k // group)
    x = torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16)
    y = aw.awq_linear(x, quant)
    rows = min(m, 64)
    w_eff = R.round_bf16(R.awq_dequantize(quant.q.cpu().numpy(), quant.group_scales.cpu().numpy(),
                                          quant.chan_scale.cpu().numpy(), group))
    _check_linear(y[:rows], R.linear_f64(x[:rows].float().cpu().numpy(), w_eff), f"awq g{group} M={m}")


def test_awq_linear_bias_fp16(aw):
    w, x32, _ = awq_layer(5, n_tokens=32)
    wt = torch.from_numpy(w).to(DEV)
    quant = aw.quantize_awq_int4(wt, x=torch.from_numpy(x32).to(DEV))
    x = torch.from_numpy(x32).to(DEV).to(torch.float16)
    bias = torch.randn(256, device=DEV).to(torch.float16)
    y = aw.awq_linear(x, quant, bias=bias)
    assert y.shape == (32, 256) and y.dtype == torch.float16
    assert torch.allclose(y - bias, aw.awq_linear(x, quant), atol=1e-2)
    w_eff = R.round_to(aw.awq_dequantize(quant).cpu().numpy(), "f16")
    _check_linear(y, R.linear_f64(x.float().cpu().numpy(), w_eff, bias.float().cpu().numpy()), "awq fp16 bias")


@pytest.mark.parametrize("param", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,k,group", [(64, 512, 128), (100, 384, 64), (7, 96, 32)])
def test_quantize_uint4_asym_bitexact(param, n, k, group):
    from scratch_llm_amd.quant import int4_group as q4

    g = torch.Generator().manual_seed(n * k)
    w = torch.randn(n, k, generator=g) * 0.05 + 0.01
    w[0, :group] = torch.rand(group, generator=g)  # all-positive group
    w[1, :group] = 0.0  # zero group
    q, s, z = q4.quantize_groupwise_uint4_asym(w.to(DEV), group, param)
    qr, sr, zr = R.quantize_groupwise_uint4_asym(w.numpy(), group, param="bf16" if param == torch.bfloat16 else "f32")
    assert np.array_equal(q.cpu().numpy(), qr)
    assert np.array_equal(bits(s.float().cpu().numpy()), bits(sr))
    assert np.array_equal(bits(z.float().cpu().numpy()), bits(zr))


@pytest.mark.parametrize("rows,cols,dtype,offset", [(2048, 4096, torch.bfloat16, 0), (64, 14336, torch.float16, 0),
                                                     (3, 100, torch.bfloat16, 0), (5, 4096, torch.bfloat16, 1)])
def test_scale_columns_bitexact(aw, rows, cols, dtype, offset):
    """sqx_scale_columns (the AWQ linear's x / s pass) is bf16/fp16(fp32 x / s) with IEEE division, bit
    for bit: the 16-byte form (cols % 8 == 0, aligned) and the element form (ragged or unaligned)."""
    from scratch_llm_amd import _lib

    print_case("scale_columns", rows, cols, dtype, offset)
    g = torch.Generator().manual_seed(rows + cols)
    x = (torch.randn(rows * cols + offset, generator=g) * 3).to(dtype)
    s = torch.exp(torch.empty(cols).uniform_(-2.0, 2.0, generator=g))
    xd, sd = x.to(DEV), s.to(DEV)
    out = torch.empty(rows * cols + offset, dtype=dtype, device=DEV)
    lib = _lib.load()
    _lib.check(lib.sqx_scale_columns(xd[offset:].data_ptr(), _lib.sqx_dtype(dtype), sd.data_ptr(), rows, cols,
                                     out[offset:].data_ptr(), _lib.stream_ptr(xd.device)), "scale_columns")
    torch.cuda.synchronize()
    want = (x[offset:].view(rows, cols).float() / s).to(dtype)
    assert torch.equal(out[offset:].cpu().view(rows, cols), want)
