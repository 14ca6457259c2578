"""FP8 E4M3 on the MI355X (fp8_weights.py W8A8 and fp8_kv_per_head.py quantizers): codes,
scales and counts bit-exact against the numpy oracle (oracle/fp8_ref.py); the W8A8 linear against
the float64 oracle within the reference's own derived bound (tests/quant/test_s1_s_r2.py:510-539):

    |got - ref| <= |ref| * eps(out_dtype) / 2 + sum|x w| * sqrt(K) * eps(fp32)

where ref and sum|x w| use the per-token-quantized activations and the dequantized weights.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
from torch import nn

from oracle import fp8_ref as F
from tests.conftest import print_case
from tests.test_oracle_fp8 import _grid

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def f8():
    from scratch_llm_amd import _lib
    from scratch_llm_amd.quant import fp8_weights

    _lib.load()
    return fp8_weights


def test_saturating_cast_bit_exact(f8):
    print_case("fp8 saturating cast")
    v = _grid()
    got = f8.saturating_cast_e4m3(torch.from_numpy(v).to(DEV)).view(torch.uint8).cpu().numpy()
    assert np.array_equal(got, F.e4m3_encode_sat(v))
    for dt in (torch.bfloat16, torch.float16):
        t = torch.from_numpy(v[np.abs(v) < 6e4]).to(dt)
        got = f8.saturating_cast_e4m3(t.to(DEV)).view(torch.uint8).cpu().numpy()
        assert np.array_equal(got, F.e4m3_encode_sat(t.float().numpy()))
    nan = f8.saturating_cast_e4m3(torch.tensor([float("nan"), 1.0], device=DEV)).view(torch.uint8).cpu()
    assert int(nan[0]) & 0x7F == 0x7F and int(nan[1]) == 0x38


@pytest.mark.parametrize("rows,cols,dtype", [(4096, 4096, torch.bfloat16), (64, 14336, torch.float32),
                                             (7, 96, torch.float16), (33, 40, torch.float32), (1, 16, torch.bfloat16)])
def test_quantize_rows_bit_exact(f8, rows, cols, dtype):
    print_case("fp8 quantize rows", rows, cols, dtype)
    g = torch.Generator().manual_seed(rows + cols)
    w = torch.randn(rows, cols, generator=g) * torch.logspace(-3, 3, rows)[:, None]
    w[0, :] = 0.0  # an all-zero row takes the MIN_SCALE floor
    w = w.to(dtype)
    codes, scale = f8.quantize_per_channel(w.to(DEV))
    assert codes.dtype == torch.float8_e4m3fn and tuple(scale.shape) == (rows, 1)
    wc, ws = F.quantize_rows(w.float().numpy())
    assert np.array_equal(codes.view(torch.uint8).cpu().numpy(), wc)
    assert np.array_equal(scale.cpu().numpy().view(np.uint32), ws.view(np.uint32))
    xc, xs = f8.quantize_per_token(w.to(DEV))
    assert torch.equal(xc.view(torch.uint8), codes.view(torch.uint8)) and torch.equal(xs, scale)
    deq = f8.dequantize(codes, scale).cpu().numpy()
    assert np.array_equal(deq.view(np.uint32), F.dequantize(wc, ws).view(np.uint32))


def test_quantize_rejects_bad_rank(f8):
    with pytest.raises(ValueError, match="weight must be 2-D"):
        f8.quantize_per_channel(torch.zeros(2, 3, 4, device=DEV))
    with pytest.raises(ValueError, match="activation must be 2-D"):
        f8.quantize_per_token(torch.zeros(5, device=DEV))


def _ref_bound(x, codes, scale, bias, out_dtype):
    """float64 oracle and the reference's derived bound, for x on the host."""
    ref = F.fp8_linear_reference(x.float().numpy(), codes.view(torch.uint8).cpu().numpy(), scale.cpu().numpy(),
                                 None if bias is None else bias.float().cpu().numpy())
    xc, xs = F.quantize_rows(x.float().numpy())
    xd = np.abs(F.e4m3_decode(xc).astype(np.float64) * xs)
    wd = np.abs(F.e4m3_decode(codes.view(torch.uint8).cpu().numpy()).astype(np.float64) * scale.cpu().numpy())
    mag = xd @ wd.T
    k = x.shape[1]
    eps_out = {torch.bfloat16: 2.0**-7, torch.float32: 2.0**-23}[out_dtype]
    bound = np.abs(ref) * eps_out / 2 + mag * math.sqrt(k) * 2.0**-23
    return ref, bound


def test_linear_reference_case(f8):
    """The reference's own GPU test case (tests/quant/test_s1_s_r2.py:520-539): seed 5, m=128, k=512,
    n=256, bf16 randn, bf16 out."""
    print_case("fp8 linear reference case")
    torch.manual_seed(5)
    x = torch.randn(128, 512, device=DEV, dtype=torch.bfloat16)
    w = torch.randn(256, 512, device=DEV, dtype=torch.bfloat16)
    codes, scale = f8.quantize_per_channel(w)
    got = f8.fp8_linear(x, codes, scale, out_dtype=torch.bfloat16).double().cpu().numpy()
    ref, bound = _ref_bound(x.cpu(), codes, scale, None, torch.bfloat16)
    assert np.all(np.abs(got - ref) <= bound), f"{float((np.abs(got - ref) / bound).max()):.3f}x the bound"


@pytest.mark.parametrize("m", [1, 4, 16, 64, 100])
@pytest.mark.parametrize("n,k", [(4096, 4096), (1024, 4096), (4096, 14336), (520, 1056), (16392, 1056), (6152, 4096)])
def test_linear_within_derived_bound(f8, m, n, k):
    """Every launch the library picks: the GEMV, and for 2..64 rows with a bf16 output the skinny
    kernel where its table says so (16392 rows: 1025 tiles, the last one half full, K with a half
    k-block at the end; 6152 rows: 385 tiles; 4096 x 14336: K split 4)."""
    print_case("fp8 linear", m, n, k)
    g = torch.Generator().manual_seed(m * 7 + n + k)
    w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    x[:, :: max(1, k // 37)] *= 20.0  # outlier channels
    codes, scale = f8.quantize_per_channel(w.to(DEV))
    bias = torch.randn(n, generator=g).to(torch.bfloat16)
    for out_dtype, b in ((torch.bfloat16, bias), (torch.float32, None)):
        got = f8.fp8_linear(x.to(DEV), codes, scale, None if b is None else b.to(DEV), out_dtype=out_dtype)
        assert got.dtype == out_dtype and got.shape == (m, n)
        ref, bound = _ref_bound(x, codes, scale, b, out_dtype)
        err = np.abs(got.double().cpu().numpy() - ref)
        assert np.all(err <= bound), f"{out_dtype}: {float((err / bound).max()):.3f}x the bound"


@pytest.mark.parametrize("m", [2, 7, 16, 33, 64])
@pytest.mark.parametrize("n,k,tiles,waves,splits", [(520, 1056, 2, 8, 1), (520, 1056, 4, 3, 4), (1000, 4104, 4, 8, 8),
                                                    (4096, 14336, 4, 8, 4), (16392, 512, 2, 4, 1), (100, 64, 4, 8, 2)])
def test_skinny_launch_shapes_within_bound(f8, m, n, k, tiles, waves, splits):
    """sqx_fp8_skinny at explicit launch shapes (tiles per workgroup, waves, K splits, including
    more splits than a wave's k-blocks allow and ragged rows and K), with a bias, within the derived
    bound; the split partials are scaled by the reduce kernel."""
    from scratch_llm_amd import _lib

    print_case("fp8 skinny", m, n, k, tiles, waves, splits)
    lib = _lib.load()
    g = torch.Generator().manual_seed(m * 5 + n + k + splits)
    w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    x[:, :: max(1, k // 37)] *= 20.0
    bias = torch.randn(n, generator=g).to(torch.bfloat16)
    codes, scale = f8.quantize_per_channel(w.to(DEV))
    tw = f8.tile_fp8(codes, scale)
    xd, bd = x.to(DEV), bias.to(DEV)
    y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
    nb = int(lib.sqx_fp8_skinny_workspace_bytes(m, n, k, splits))
    ws = torch.empty(-(-nb // 4), dtype=torch.float32, device=DEV)
    _lib.check(lib.sqx_fp8_skinny(tw.wt.data_ptr(), tw.scale.data_ptr(), xd.data_ptr(), _lib.DTYPE_BF16, y.data_ptr(),
                                  bd.data_ptr(), m, n, k, tiles, waves, splits, ws.data_ptr(), nb,
                                  _lib.stream_ptr(torch.device(DEV))), "sqx_fp8_skinny")
    ref, bound = _ref_bound(x, codes, scale, bias, torch.bfloat16)
    err = np.abs(y.double().cpu().numpy() - ref)
    assert np.all(err <= bound), f"{float((err / bound).max()):.3f}x the bound"
    # a workspace one split short is refused before any launch
    if splits > 1 and nb > int(lib.sqx_fp8_skinny_workspace_bytes(m, n, k, 1)):
        assert lib.sqx_fp8_skinny(tw.wt.data_ptr(), tw.scale.data_ptr(), xd.data_ptr(), _lib.DTYPE_BF16, y.data_ptr(),
                                  None, m, n, k, tiles, waves, splits, ws.data_ptr(), nb - 4,
                                  _lib.stream_ptr(torch.device(DEV))) != 0


def test_skinny_refusals(f8):
    from scratch_llm_amd import _lib

    lib = _lib.load()
    codes, scale = f8.quantize_per_channel(torch.randn(64, 128, device=DEV))
    tw = f8.tile_fp8(codes, scale)
    x = torch.randn(65, 128, device=DEV).to(torch.bfloat16)
    y = torch.empty(65, 64, dtype=torch.bfloat16, device=DEV)
    ws = torch.empty(1 << 20, dtype=torch.uint8, device=DEV)
    s = _lib.stream_ptr(torch.device(DEV))

    def call(m, tiles, waves, splits):
        return lib.sqx_fp8_skinny(tw.wt.data_ptr(), tw.scale.data_ptr(), x.data_ptr(), _lib.DTYPE_BF16, y.data_ptr(),
                                  None, m, 64, 128, tiles, waves, splits, ws.data_ptr(), ws.numel(), s)

    assert call(65, 2, 8, 1) != 0  # more than 64 rows
    assert call(4, 3, 8, 1) != 0  # tiles must be 2 or 4
    assert call(4, 2, 9, 1) != 0  # at most 8 waves
    assert call(4, 2, 8, 0) != 0  # at least one split
    assert call(4, 2, 8, 1) == 0


def test_linear_shapes_and_refusals(f8):
    w = torch.randn(32, 48, device=DEV)
    codes, scale = f8.quantize_per_channel(w)
    x = torch.randn(2, 3, 48, device=DEV)
    y = f8.fp8_linear(x, codes, scale)
    assert y.shape == (2, 3, 32) and y.dtype == torch.bfloat16
    with pytest.raises(ValueError, match="activation last dim 40 != weight K 48"):
        f8.fp8_linear(torch.randn(2, 40, device=DEV), codes, scale)
    c2, s2 = f8.quantize_per_channel(torch.randn(8, 40, device=DEV))
    with pytest.raises(ValueError, match="K % 16 == 0, got K=40"):
        f8.fp8_linear(torch.randn(2, 40, device=DEV), c2, s2)
    with pytest.raises(RuntimeError):
        f8.fp8_linear(torch.randn(2, 48), codes, scale)


class _Block(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.up = nn.Linear(256, 512)
        self.down = nn.Linear(512, 256, bias=False)
        self.odd = nn.Linear(40, 8)  # in_features % 16 != 0: left alone


class _Toy(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.blocks = nn.ModuleList([_Block(), _Block()])
        self.lm_head = nn.Linear(256, 64)


def test_module_and_converter(f8):
    """Fp8Linear / convert_linears_to_fp8 (fp8_weights.py:289-400): names replaced, skips, forward."""
    print_case("fp8 module")
    torch.manual_seed(9)
    model = _Toy().to(DEV).to(torch.bfloat16)
    names = f8.convert_linears_to_fp8(model)
    assert names == ["blocks.0.up", "blocks.0.down", "blocks.1.up", "blocks.1.down"]
    assert isinstance(model.lm_head, nn.Linear) and isinstance(model.blocks[0].odd, nn.Linear)
    mod = model.blocks[0].up
    assert mod.weight_codes.dtype == torch.float8_e4m3fn and mod.weight_codes.element_size() == 1
    assert mod.out_dtype == torch.bfloat16
    x = torch.randn(5, 256, device=DEV).to(torch.bfloat16)
    y = mod(x)
    ref, bound = _ref_bound(x.cpu(), mod.weight_codes, mod.weight_scale, mod.bias, torch.bfloat16)
    assert np.all(np.abs(y.double().cpu().numpy() - ref) <= bound)
    wd = mod.dequantized_weight()
    assert torch.equal(wd, f8.dequantize(mod.weight_codes, mod.weight_scale))
    with pytest.raises(RuntimeError):
        mod(torch.randn(2, 256))


def test_per_head_kv_quantizers_bit_exact():
    print_case("fp8 per-head")
    from scratch_llm_amd.quant import fp8_kv_per_head as K

    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 8, 33, 128, generator=g) * torch.logspace(-3, 3, 8).view(1, 8, 1, 1)
    x[1] *= 2.0
    xd = x.to(DEV)
    amax = K.per_head_amax(xd)
    scale = K.per_head_scale(xd)
    assert tuple(scale.shape) == (1, 8, 1, 1)
    assert np.array_equal(amax.cpu().numpy(), F.per_head_amax(x.numpy()))
    assert np.array_equal(scale.cpu().numpy().view(np.uint32), F.per_head_scale(x.numpy()).view(np.uint32))
    codes = K.quantize_per_head(xd, scale)
    assert np.array_equal(codes.view(torch.uint8).cpu().numpy(), F.quantize_per_head(x.numpy(), scale.cpu().numpy()))
    deq = K.dequantize_per_head(codes, scale)
    assert np.array_equal(deq.cpu().numpy(), F.dequantize_per_head(F.quantize_per_head(x.numpy(), scale.cpu().numpy()),
                                                                    scale.cpu().numpy()))
    over = x.clone()
    over[:, 0] = over[:, 0].abs().clamp_min(1.0) * 1e4
    assert K.saturated_count(over.to(DEV), scale) == F.saturated_count(over.numpy(), scale.cpu().numpy()) > 0
    with pytest.raises(ValueError, match="not per-head"):
        K.quantize_per_head(xd, scale.expand(2, -1, -1, -1))


def _kv_block(batch=2, heads=4, tokens=16, dim=32, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, heads, tokens, dim, generator=g)
    return (x * torch.logspace(-2, 2, heads).view(1, heads, 1, 1)).to(DEV)


def test_per_head_cache_contract():
    """PerHeadFp8KVCache on the device: the decode contract and the laws the reference's tests state
    (tests/quant/test_s1_s_r2.py:278-400): calibration on the first block, saturation counted and
    landing on 448 * scale, one byte per element plus the scales once, installed scales used as given,
    growth across appends keeps every stored code."""
    from scratch_llm_amd.quant import fp8_kv_per_head as K

    print_case("fp8 per-head cache")
    cache = K.PerHeadFp8KVCache(n_layers=2)
    assert cache.length == 0 and cache.get(0) is None and cache.codes(1) is None
    assert cache.scales(0) == (None, None) and cache.saturated_fraction() == 0.0
    x = _kv_block()
    cache.append(0, x, x)
    cache.advance(x.shape[2])
    k_scale, v_scale = cache.scales(0)
    assert torch.equal(k_scale, K.per_head_scale(x)) and torch.equal(v_scale, K.per_head_scale(x))
    assert cache.k_saturated == 0 and cache.v_saturated == 0  # the calibration block fits its own amax
    k_out, v_out = cache.get(0)
    assert k_out.shape == x.shape and k_out.dtype == torch.float32
    assert torch.equal(k_out, K.dequantize_per_head(K.quantize_per_head(x, k_scale), k_scale))
    # a block past the calibrated range saturates, is counted, and lands on the top of the head's range
    over = x[:, :, :1].clone()
    over[:, 0] = over[:, 0].abs().clamp_min(1.0) * 1e4
    n_over = K.saturated_count(over, k_scale)
    assert n_over > 0
    cache.append(0, over, over)
    cache.advance(1)
    assert cache.length == x.shape[2] + 1
    assert cache.k_saturated == n_over and cache.v_saturated == n_over and cache.saturated_fraction() > 0
    k_out, _ = cache.get(0)
    assert not torch.isnan(k_out).any()
    assert torch.allclose(k_out[:, 0, -1].abs(), torch.full_like(k_out[:, 0, -1], 448.0 * float(k_scale[0, 0, 0, 0])))
    # many small appends grow the buffer and keep every code (the concatenation of the blocks)
    blocks = [_kv_block(tokens=t, seed=10 + t) for t in (1, 3, 1, 40, 2)]
    for b in blocks:
        cache.append(1, b, -b)
    codes_k, codes_v = cache.codes(1)
    assert codes_k.dtype == torch.float8_e4m3fn and codes_k.element_size() == 1
    ks, vs = cache.scales(1)
    want_k = torch.cat([K.quantize_per_head(b, ks) for b in blocks], dim=2)
    want_v = torch.cat([K.quantize_per_head(-b, vs) for b in blocks], dim=2)
    assert torch.equal(codes_k.view(torch.uint8), want_k.view(torch.uint8))
    assert torch.equal(codes_v.view(torch.uint8), want_v.view(torch.uint8))
    n_el = 2 * (x.numel() + over.numel()) + 2 * sum(b.numel() for b in blocks)
    assert cache.kv_bytes == n_el + 2 * 2 * x.shape[1] * 4
    assert cache.kv_bytes < K.bf16_reference_bytes(n_el)
    with pytest.raises(ValueError, match="holds blocks"):
        cache.append(1, _kv_block(dim=64), _kv_block(dim=64))
    # installed scales take precedence over calibration
    c2 = K.PerHeadFp8KVCache(n_layers=1)
    one = torch.ones(1, x.shape[1], 1, 1, device=DEV)
    c2.set_scales(0, one, one)
    c2.append(0, x * 10, x * 10)  # the loud heads pass 448 at scale 1
    assert torch.equal(c2.scales(0)[0], one) and c2.k_saturated > 0
    with pytest.raises(ValueError, match=r"\(1, H, 1, 1\)"):
        c2.set_scales(0, one.view(-1), one)
    # codes() and scales() hand out copies, as the reference's torch.cat and replaced scale tensors:
    # a 16-token block fills the first buffer exactly, where a view would alias the storage
    c3 = K.PerHeadFp8KVCache(n_layers=1)
    c3.append(0, x, x)
    before = c3.get(0)[0].clone()
    ck, cv = c3.codes(0)
    ck.view(torch.uint8).fill_(0)
    cv.view(torch.uint8).fill_(0x7E)
    assert torch.equal(c3.get(0)[0], before)
    old_k, _ = c3.scales(0)
    kept = old_k.clone()
    c3.set_scales(0, one * 3, one * 3)
    assert torch.equal(old_k, kept) and torch.equal(c3.scales(0)[0], one * 3)
