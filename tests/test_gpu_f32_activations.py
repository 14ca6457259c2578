"""fp32 activations in the int4 and AWQ linears (``w4a16_linear`` and ``awq_linear`` accept any
``x.dtype`` and run ``F.linear`` in fp32, int4_group.py:157-164, awq.py:184-192).

The library runs x as three bf16 rows (``a = bf16(x)``, ``b = bf16(x - a)``, ``c = bf16(x - a - b)``,
whose sum is x exactly for normal fp32 values) through the int4 decode GEMV with fp32 outputs and
adds them (``sqx_int4_linear_f32``). Against the float64 product of x and the fp32 dequantized weight
(no bf16 rounding of the weight, as the reference's fp32 F.linear) each output is within
``2**-17 * sum_k |x_k w_k|``: the code products are exact, the fp32 accumulation of each part adds at
most (K/32 + 8) * 2**-24 of its sum of magnitudes, and the final adds two fp32 roundings. Plus the
north star's max-abs-rel 1e-2; the reference's own law awq_linear(x) == x @ awq_dequantize(quant).T
to 1e-5 (tests/test_quant_awq.py:130-137) is checked on the GPU in tests/test_gpu_awq.py.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import quant_ref as R
from tests.conftest import print_case

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def mods():
    from scratch_llm_amd import _lib
    from scratch_llm_amd.quant import awq, int4_group

    _lib.load()
    return int4_group, awq


def _check_f32(y: torch.Tensor, x: np.ndarray, w: np.ndarray, bias: np.ndarray | None, what: str) -> None:
    assert y.dtype == torch.float32
    xd, wd = x.astype(np.float64), w.astype(np.float64)
    y_ref = xd @ wd.T
    mag = np.abs(xd) @ np.abs(wd).T
    if bias is not None:
        y_ref = y_ref + bias[None, :]
        mag = mag + np.abs(bias)[None, :]
    yv = y.cpu().numpy().astype(np.float64)
    assert np.isfinite(yv).all(), f"{what}: non-finite output"
    err = np.abs(yv - y_ref)
    assert float(err.max() / np.abs(y_ref).max()) <= 1e-2, f"{what}: max-abs-rel"
    worst = float((err / (2.0**-17 * mag + 1e-30)).max())
    assert worst <= 1.0, f"{what}: {worst:.2f}x the fp32-activation bound"


@pytest.mark.parametrize("n,k,group,m", [(4096, 4096, 128, 1), (1000, 1024, 128, 5), (256, 512, 64, 32),
                                         (300, 384, 32, 33), (512, 4096, 128, 100), (64, 256, 128, 1)])
def test_w4a16_linear_fp32_x(mods, n, k, group, m):
    i4, _ = mods
    print_case("w4a16 fp32 x", n, k, group, m)
    g = torch.Generator(device=DEV).manual_seed(n + k + m)
    w = torch.randn(n, k, generator=g, device=DEV) * 0.02
    q, s = i4.quantize_groupwise_int4(w, group)
    x = torch.randn(2, m, k, generator=g, device=DEV) * 3.0
    bias = torch.randn(n, generator=g, device=DEV)
    y = i4.w4a16_linear(x, q, s, bias=bias, group_size=group)
    assert y.shape == (2, m, n)
    w_eff = R.dequantize_groupwise_int4(q.cpu().numpy(), s.cpu().numpy(), group)
    _check_f32(y.reshape(-1, n), x.reshape(-1, k).cpu().numpy(), w_eff, bias.cpu().numpy(), f"{k}->{n} g{group} M={m}")
    y0 = i4.w4a16_linear(x, q, s, group_size=group)
    _check_f32(y0.reshape(-1, n), x.reshape(-1, k).cpu().numpy(), w_eff, None, "no bias")


def test_asymmetric_fp32_x(mods):
    i4, _ = mods
    n, k = 1024, 4096
    g = torch.Generator(device=DEV).manual_seed(77)
    w = torch.randn(n, k, generator=g, device=DEV) * 0.02
    qa, sa, za = i4.quantize_groupwise_uint4_asym(w, 128, torch.bfloat16)
    tw = i4.tile_int4(qa, sa, za, 128)
    w_eff = R.dequantize_groupwise_uint4_asym(qa.cpu().numpy(), sa.float().cpu().numpy(), za.float().cpu().numpy())
    for m in (1, 8, 70):
        x = torch.randn(m, k, generator=g, device=DEV)
        _check_f32(i4.int4_linear_tiled_f32(x, tw), x.cpu().numpy(), w_eff, None, f"asym M={m}")


@pytest.mark.parametrize("m", [1, 16, 200])
def test_awq_linear_fp32_x(mods, m):
    _, aw = mods
    n, k = 1024, 4096
    print_case("awq fp32 x", m)
    g = torch.Generator(device=DEV).manual_seed(500 + m)
    w = torch.randn(n, k, generator=g, device=DEV) * 0.02
    sc = torch.exp(torch.empty(k, device=DEV).uniform_(np.log(0.5), np.log(2.0), generator=g))
    quant = aw.quantize_awq_int4(w, chan_scale=sc)
    x = torch.randn(m, k, generator=g, device=DEV)
    x[:, :40] *= 20.0
    y = aw.awq_linear(x, quant)
    _check_f32(y, x.cpu().numpy(), aw.awq_dequantize(quant).cpu().numpy(), None, f"awq fp32 M={m}")


def test_wide_groups_and_unsupported_group_and_dtype(mods):
    """A group of 256 runs as two 128-column groups with the scale repeated: bit for bit the linear of
    the repeated scales, fp32 activations included; a group that is not a multiple of 32 raises, and
    so does a float64 activation."""
    i4, aw = mods
    w = torch.randn(16, 512, device=DEV) * 0.02
    x = torch.randn(3, 512, device=DEV)
    q, s = i4.quantize_groupwise_int4(w, 256)
    y = i4.w4a16_linear(x, q, s, group_size=256)
    assert torch.equal(y, i4.w4a16_linear(x, q, s.repeat_interleave(2, dim=1).contiguous(), group_size=128))
    q48, s48 = i4.quantize_groupwise_int4(w[:, :480], 48)
    with pytest.raises(ValueError, match="group_size=48"):
        i4.w4a16_linear(x[:, :480], q48, s48, group_size=48)
    q, s = i4.quantize_groupwise_int4(w)
    with pytest.raises(TypeError):
        i4.w4a16_linear(torch.randn(1, 512, device=DEV, dtype=torch.float64), q, s)
    quant = aw.quantize_awq_int4(w, chan_scale=torch.ones(512, device=DEV), group_size=256)
    ya = aw.awq_linear(x, quant)
    q2 = aw.AWQQuant(q=quant.q, group_scales=quant.group_scales.repeat_interleave(2, dim=1).contiguous(),
                     chan_scale=quant.chan_scale, group_size=128)
    assert torch.equal(ya, aw.awq_linear(x, q2))
    quant48 = aw.quantize_awq_int4(w[:, :480], chan_scale=torch.ones(480, device=DEV), group_size=48)
    with pytest.raises(ValueError, match="group_size=48"):
        aw.awq_linear(x[:, :480], quant48)
