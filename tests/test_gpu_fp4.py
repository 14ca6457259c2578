"""FP4 parity on the MI355X: the HIP kernels (through libsqx_hip.so) against the numpy oracle.

Bit-exact: E2M1 round/decode, pack/unpack, E4M3/E8M0 codecs, MXFP4 / NVFP4 quantize (codes, block
scales, global scale) and dequantize, including the reference's own golden vectors.
Linears: max|y - y_ref| / max|y_ref| <= 1e-2 against the float64 product of x and the dequantized
weight rounded to the activation dtype (the reference's ``.to(x.dtype)``), plus the elementwise
bound |y - y_ref| <= 2**-7 (|y_ref| + rms(y_ref)). The fp32-activation NVFP4 linear follows the
reference's law (rel Frobenius < 1e-4 against the fp32 dequant-matmul, test_quant_nvfp4_mxfp4.py:183-193).
"""

from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import quant_ref as R
from tests.conftest import print_case

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLDEN = Path(__file__).resolve().parent / "golden" / "reference_vectors.json"


@pytest.fixture(scope="module")
def f4():
    from scratch_llm_amd import _lib
    from scratch_llm_amd.quant import nvfp4_mxfp4

    _lib.load()
    return nvfp4_mxfp4


@pytest.fixture(scope="module")
def ref_vectors() -> dict:
    return json.loads(GOLDEN.read_text())


def f32(hexes) -> np.ndarray:
    return np.array([struct.unpack("<f", bytes.fromhex(h))[0] for h in hexes], np.float32)


def bits(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, np.float32)).view(np.uint32)


def dev(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _check_linear(y_gpu: torch.Tensor, y_ref: np.ndarray, what: str) -> float:
    y = y_gpu.float().cpu().numpy().astype(np.float64)
    assert np.isfinite(y).all(), f"{what}: non-finite output"
    err = np.abs(y - y_ref)
    scale = np.abs(y_ref).max()
    rel = float(err.max() / scale) if scale > 0 else float(err.max())
    rms = float(np.sqrt((y_ref**2).mean()))
    worst = float((err / (2.0**-7 * (np.abs(y_ref) + rms) + 1e-30)).max())
    assert rel <= 1e-2, f"{what}: max-abs-rel {rel:.3e} > 1e-2"
    assert worst <= 1.0, f"{what}: elementwise bound exceeded by {worst:.2f}x"
    return rel


def _random_values(n: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(n) * rng.choice([1e-3, 0.05, 1.0, 7.0, 300.0], n)).astype(np.float32)
    # exact midpoints, grid values and signed zeros scaled by powers of two
    grid = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 0.5, 6.0, -0.0, 0.0], np.float32)
    pattern = np.tile(grid, 4) * np.repeat(np.float32([1, -1, 0.5, 4]), grid.size)
    k = min(n, pattern.size)
    x[:k] = pattern[:k]
    return x


# ------------------------------------------------------------------------------------ codecs
def test_e2m1_round_and_decode_bitexact(f4, ref_vectors):
    x = _random_values(100_003, 1)
    c = f4.e2m1_round_to_code(dev(x)).cpu().numpy()
    assert np.array_equal(c, R.e2m1_round_to_code(x))
    g = ref_vectors["e2m1_specials"]
    assert f4.e2m1_round_to_code(dev(f32(g["x"]))).cpu().tolist() == g["codes"]
    codes = np.arange(16, dtype=np.uint8)
    assert np.array_equal(bits(f4.e2m1_decode(dev(codes)).cpu().numpy()), bits(R.e2m1_decode(codes)))
    # bf16 / fp16 inputs are converted exactly to fp32 first
    xb = torch.from_numpy(x).to(torch.bfloat16)
    assert np.array_equal(f4.e2m1_round_to_code(xb.to(DEV)).cpu().numpy(), R.e2m1_round_to_code(xb.float().numpy()))


def test_e2m1_round_boundaries_bitexact(f4):
    """The device rounding decides by comparisons with the midpoints below 2**22 and by fp32
    distances above: every value within 64 ulps of each midpoint, each magnitude and each power of two
    from 2**18 to 2**30 (the switch and the range where the reference's distances round), both signs,
    plus subnormals and specials, against the oracle's argmin."""
    anchors = np.float32([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0] +
                         [2.0**e for e in range(18, 31)] + [3.0 * 2.0**e for e in range(18, 30)])
    bits_ = anchors.view(np.int32)[:, None] + np.arange(-64, 65, dtype=np.int32)[None, :]
    x = bits_.reshape(-1).view(np.float32)
    sub = np.arange(1, 4096, dtype=np.int32).view(np.float32)
    specials = np.float32([np.inf, np.nan, 0.0, np.finfo(np.float32).max, np.finfo(np.float32).tiny])
    x = np.concatenate([x, sub, specials])
    x = np.concatenate([x, -x])
    c = f4.e2m1_round_to_code(dev(x)).cpu().numpy()
    want = R.e2m1_round_to_code(x)
    bad = np.flatnonzero(c != want)
    assert bad.size == 0, f"{bad.size} codes differ, first at x={x[bad[0]]!r}: {c[bad[0]]} vs {want[bad[0]]}"


@pytest.mark.parametrize("n", [1, 2, 3, 17, 4096, 4097, 1 << 20])
def test_fp4_pack_unpack_bitexact(f4, n):
    rng = np.random.default_rng(n)
    c = rng.integers(0, 16, n).astype(np.uint8)
    p = f4.pack_fp4(dev(c))
    assert np.array_equal(p.cpu().numpy(), R.pack_fp4(c))
    assert np.array_equal(f4.unpack_fp4(p, n).cpu().numpy(), c)


def test_scale_codecs_bitexact(f4, ref_vectors, known_answers):
    rng = np.random.default_rng(3)
    v = np.abs(rng.standard_normal(50_000) * rng.choice([1e-4, 1e-2, 1, 30, 500], 50_000)).astype(np.float32)
    v[:5] = [0.0, -1.0, np.nan, np.inf, 1e-42]
    assert np.array_equal(bits(f4.quantize_e4m3(dev(v)).cpu().numpy()), bits(R.quantize_e4m3(v)))
    assert np.array_equal(bits(f4.quantize_e8m0(dev(v)).cpu().numpy()), bits(R.quantize_e8m0(v)))
    g = ref_vectors["e4m3_edges"]
    assert np.array_equal(bits(f4.quantize_e4m3(dev(f32(g["v"]))).cpu().numpy()), bits(f32(g["out"])))
    g = ref_vectors["e8m0_midpoints"]
    assert np.array_equal(bits(f4.quantize_e8m0(dev(f32(g["v"]))).cpu().numpy()), bits(f32(g["out"])))


# ------------------------------------------------------------------------------------ quantize
@pytest.mark.parametrize("shape,block,dtype", [
    ((64, 256), 32, torch.float32), ((37, 96), 32, torch.bfloat16), ((1000,), 32, torch.float32),
    ((128, 512), 16, torch.float32), ((8, 128), 64, torch.float16), ((3, 7), 32, torch.float32),
])
def test_mxfp4_quantize_bitexact(f4, shape, block, dtype):
    print_case("mxfp4 quantize", shape, block, dtype)
    n = int(np.prod(shape))
    x = torch.from_numpy(_random_values(n, n).reshape(shape)).to(dtype)
    q = f4.mxfp4_quantize(x.to(DEV), block)
    codes, s_block, _, _, _ = R.mxfp4_quantize(x.float().numpy(), block)
    assert np.array_equal(q.codes.cpu().numpy(), codes)
    assert np.array_equal(bits(q.s_block.cpu().numpy()), bits(s_block))
    assert q.n == n and tuple(q.shape) == shape and q.block == block
    d = f4.mxfp4_dequantize(q).cpu().numpy()
    assert np.array_equal(bits(d), bits(R.mxfp4_dequantize(codes, s_block, shape, n)))


def test_mxfp4_scale_edges_golden(f4, ref_vectors):
    g = ref_vectors["mxfp4_scale_edges"]
    rows = g["rows"]
    x = np.zeros((rows, 32), np.float32)
    x[:, :5] = f32(g["x_head"]).reshape(rows, 5)
    q = f4.mxfp4_quantize(dev(x), 32)
    assert np.array_equal(bits(q.s_block.cpu().numpy()), bits(f32(g["s_block"])))
    assert q.codes[:, :5].reshape(-1).cpu().tolist() == g["codes_head"]


def test_mxfp4_scale_mantissa_sweep(f4):
    """The block exponent takes the correctly rounded fp32 log2 only when amax / 6 has a mantissa of
    1..63 and reads the float's exponent otherwise: blocks whose amax / 6 lands on every mantissa
    0..80 and the top 80 below the next power of two, at exponents -99..127, against the oracle's
    log2 form (E8M0 scales and codes)."""
    e = np.arange(-99, 128, dtype=np.int64)
    m = np.concatenate([np.arange(0, 81), np.arange(2**23 - 80, 2**23)]).astype(np.int64)
    t = (((e[:, None] + 127) << 23) | m[None, :]).astype(np.uint32).view(np.float32).reshape(-1)
    with np.errstate(over="ignore"):  # the top binade's amax overflows and is dropped
        amax = (t.astype(np.float64) * 6.0).astype(np.float32)  # amax / 6 rounds to t or a neighbour of it
    amax = amax[np.isfinite(amax)]
    x = np.zeros((amax.size, 32), np.float32)
    x[:, 0] = amax
    x[:, 1] = -amax * np.float32(0.3)
    print_case("mxfp4 scale mantissa sweep", amax.size)
    q = f4.mxfp4_quantize(dev(x), 32)
    codes, s_block, _, _, _ = R.mxfp4_quantize(x, 32)
    assert np.array_equal(bits(q.s_block.cpu().numpy()), bits(s_block))
    assert np.array_equal(q.codes.cpu().numpy(), codes)


@pytest.mark.parametrize("shape,block", [((64, 256), 16), ((1024, 48), 16), ((33, 96), 32), ((999,), 16)])
def test_nvfp4_quantize_bitexact(f4, shape, block):
    print_case("nvfp4 quantize", shape, block)
    n = int(np.prod(shape))
    x = _random_values(n, 7 + n).reshape(shape)
    q = f4.nvfp4_quantize(dev(x), block)
    codes, s_global, s_block, _, _ = R.nvfp4_quantize(x, block)
    assert np.array_equal(q.codes.cpu().numpy(), codes)
    assert np.array_equal(bits(q.s_block.cpu().numpy()), bits(s_block))
    assert bits(q.s_global.cpu().numpy().reshape(1))[0] == bits(np.float32(s_global).reshape(1))[0]
    d = f4.nvfp4_dequantize(q).cpu().numpy()
    assert np.array_equal(bits(d), bits(R.nvfp4_dequantize(codes, s_global, s_block, shape, n)))


def test_small_tensors_golden(f4, ref_vectors):
    g = ref_vectors["nvfp4_small"]
    q = f4.nvfp4_quantize(dev(f32(g["x"]).reshape(g["shape"])), 16)
    assert q.codes.reshape(-1).cpu().tolist() == g["codes"]
    assert np.array_equal(bits(q.s_block.cpu().numpy()), bits(f32(g["s_block"])))
    assert bits(q.s_global.cpu().numpy().reshape(1))[0] == bits(f32([g["s_global"]]))[0]
    g = ref_vectors["mxfp4_small"]
    q = f4.mxfp4_quantize(dev(f32(g["x"]).reshape(g["shape"])), 32)
    assert q.codes.reshape(-1).cpu().tolist() == g["codes"]
    assert np.array_equal(bits(q.s_block.cpu().numpy()), bits(f32(g["s_block"])))


def test_recorded_sqnr_on_gpu(f4, known_answers):
    """bench/RESULTS.md:561 recomputed from the GPU kernels' dequantized tensors."""
    ka = known_answers["nvfp4_vs_mxfp4"]
    torch.manual_seed(ka["seed"])
    x = torch.randn(*ka["shape"]).to(DEV)
    nv = f4.nvfp4_dequantize(f4.nvfp4_quantize(x, 16))
    mx = f4.mxfp4_dequantize(f4.mxfp4_quantize(x, 32))
    xn = x.cpu().numpy()
    assert abs(R.sqnr_db(xn, nv.cpu().numpy()) - ka["nvfp4_db"]) < ka["tolerance_db"]
    assert abs(R.sqnr_db(xn, mx.cpu().numpy()) - ka["mxfp4_db"]) < ka["tolerance_db"]


# ------------------------------------------------------------------------------------ linears
CONFIG4 = [(28672, 8192), (8192, 28672)]  # (out N, in K) Llama-3-70B MLP


@pytest.fixture(scope="module", params=CONFIG4, ids=lambda s: f"{s[1]}to{s[0]}")
def mx_weight(request, f4):
    n, k = request.param
    print_case("mxfp4 weight", n, k)
    g = torch.Generator(device=DEV).manual_seed(1000 + n % 97)
    w = torch.randn(n, k, generator=g, device=DEV) * 0.02
    q = f4.mxfp4_quantize(w, 32)
    # the quantizer is pinned bit-exact elsewhere; re-check the first 16 rows of this weight here
    codes, s_block, _, _, _ = R.mxfp4_quantize(w[:16].cpu().numpy(), 32)
    assert np.array_equal(q.codes[: 16 * k // 32].cpu().numpy(), codes)
    assert np.array_equal(bits(q.s_block[: 16 * k // 32].cpu().numpy()), bits(s_block))
    del w
    # the reference's GEMM operand: dequantized weight cast to bf16 (exact here: e2m1 * 2**e)
    w_eff = f4.mxfp4_dequantize(q).to(torch.bfloat16).float().cpu().numpy()
    return n, k, q, w_eff


@pytest.mark.parametrize("m", [1, 4, 8, 128])
def test_mxfp4_linear_config4(f4, mx_weight, m):
    n, k, q, w_eff = mx_weight
    print_case("mxfp4 linear", n, k, m)
    g = torch.Generator(device=DEV).manual_seed(2000 + m)
    x = torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16)
    y = f4.mxfp4_linear(x, q)
    torch.cuda.synchronize()
    _check_linear(y, R.linear_f64(x.float().cpu().numpy(), w_eff), f"mxfp4 {k}->{n} M={m}")


@pytest.mark.parametrize("n,k,m,dtype,block", [
    (1000, 1024, 1, torch.bfloat16, 32), (40, 96, 5, torch.float16, 32), (48, 256, 17, torch.bfloat16, 64),
    (64, 4096, 64, torch.bfloat16, 32), (16, 32, 3, torch.bfloat16, 32), (300, 2048, 8, torch.float16, 32),
])
def test_mxfp4_linear_ragged(f4, n, k, m, dtype, block):
    print_case("mxfp4 ragged", n, k, m, dtype, block)
    g = torch.Generator(device=DEV).manual_seed(n * k + m)
    w = torch.randn(n, k, generator=g, device=DEV) * 0.05
    q = f4.mxfp4_quantize(w, block)
    x = torch.randn(m, k, generator=g, device=DEV).to(dtype)
    bias = torch.randn(n, generator=g, device=DEV).to(dtype)
    y = f4.mxfp4_linear(x, q, bias)
    assert y.dtype == dtype and y.shape == (m, n)
    act = "bf16" if dtype == torch.bfloat16 else "f16"
    w_eff = R.round_to(f4.mxfp4_dequantize(q).cpu().numpy(), act)
    _check_linear(y, R.linear_f64(x.float().cpu().numpy(), w_eff, bias.float().cpu().numpy()), f"{k}->{n} M={m}")


def test_mxfp4_tile_from_e8m0_bytes_matches(f4):
    """The on-disk form (packed codes + E8M0 bytes, k3/checkpoint.py:92-144) tiles identically."""
    from scratch_llm_amd import _lib

    w = torch.randn(100, 256, device=DEV) * 0.03
    q = f4.mxfp4_quantize(w, 32)
    a = f4.tile_fp4(q)
    packed = f4.pack_fp4(q.codes.reshape(-1))
    e8 = (torch.log2(q.s_block).round().to(torch.int32) + 127).to(torch.uint8).reshape(100, 8)
    lib = _lib.load()
    wt = torch.empty_like(a.wt)
    st = torch.empty_like(a.st)
    _lib.check(lib.sqx_fp4_tile(packed.data_ptr(), 1, e8.data_ptr(), _lib.FP4_SCALE_MX_E8M0, 32, 100, 256,
                                wt.data_ptr(), st.data_ptr(), _lib.stream_ptr(w.device)), "tile")
    assert torch.equal(wt, a.wt) and torch.equal(st, a.st)


@pytest.mark.parametrize("m,k,n", [(1, 4096, 4096), (8, 8192, 1024), (64, 512, 256)])
def test_nvfp4_linear_bf16(f4, m, k, n):
    print_case("nvfp4 linear", m, k, n)
    g = torch.Generator(device=DEV).manual_seed(m + k + n)
    w = torch.randn(n, k, generator=g, device=DEV) * 0.02
    q = f4.nvfp4_quantize(w, 16)
    x = torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16)
    y = f4.nvfp4_linear(x, q)
    w_eff = R.round_bf16(f4.nvfp4_dequantize(q).cpu().numpy())
    _check_linear(y, R.linear_f64(x.float().cpu().numpy(), w_eff), f"nvfp4 {k}->{n} M={m}")


def test_quant_linear_nvfp4_fp32_law(f4):
    """The reference's own laws for quant_linear_nvfp4 on its test data (tests/test_quant_nvfp4_mxfp4.py:183-215)."""
    torch.manual_seed(4)
    x = torch.randn(64, 512)
    w = torch.randn(256, 512)
    y = f4.quant_linear_nvfp4(x.to(DEV), w.to(DEV), 16)
    assert y.dtype == torch.float32 and y.shape == (64, 256)
    y_ref = R.quant_linear_nvfp4(x.numpy(), w.numpy(), 16)
    yn = y.cpu().numpy().astype(np.float64)
    assert np.linalg.norm(yn - y_ref) / np.linalg.norm(y_ref) < 1e-4
    with pytest.raises(ValueError, match="multiple of block"):
        f4.quant_linear_nvfp4(torch.randn(4, 30, device=DEV), torch.randn(8, 30, device=DEV), 16)


def test_fp4_rejects_cpu(f4):
    with pytest.raises(RuntimeError, match="device tensors"):
        f4.mxfp4_quantize(torch.randn(4, 32))
