"""MXFP4 x MXFP4 GEMM parity on the MI355X (config 4, MXFP4-activation variant).

* ``mxfp4_quantize_tiled`` is bit-exact: its tiled codes and E8M0 bytes equal the oracle's
  ``mxfp4_quantize`` of each activation row, re-laid by the tile layout restated here in numpy.
* ``mxfp4_gemm`` against the float64 product of the two oracle-dequantized operands
  (``F.linear(mxfp4_dequantize(x_q), mxfp4_dequantize(W_q))``). Every product of two dequantized
  values is exact, so the only differences are fp32 accumulation and the output rounding. The
  accumulator takes one rounded 64-term partial per MFMA k-step, each rounding at most 2**-24 of a
  partial sum bounded by ``sum_k |x_k w_k|``; the bound allows two roundings per step:
  ``(k/32 + 8) * 2**-24 * sum_k |x_k w_k|`` for fp32 output, plus half an output ulp for bf16/fp16,
  and the usual linear bar (max-abs-rel <= 1e-2, elementwise 2**-7 (|y| + rms y)).
* Full config-4 shapes (4096 x 8192 -> 28672 and 4096 x 28672 -> 8192): a sample of rows and
  columns against the oracle (quantizing a subset of rows gives the same codes, blocks are per row).
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
def f4():
    from scratch_llm_amd import _lib
    from scratch_llm_amd.quant import nvfp4_mxfp4

    _lib.load()
    return nvfp4_mxfp4


def tile_mx_np(codes: np.ndarray, e8m0: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """The tiled FP4 layout: block (t, kb) is 1 KiB, lane L owns 16 bytes holding the 32 codes of row
    16t + (L & 15), columns 128kb + 32(L >> 4) + e, two per byte, even element in the low nibble;
    scale byte L of block (t, kb) is that lane's E8M0 byte. Padding holds code 0 and byte 0."""
    m, k = codes.shape
    T, KB = -(-m // 16), -(-k // 128)
    c = np.zeros((T * 16, KB * 128), np.uint8)
    c[:m, :k] = codes
    c = c.reshape(T, 16, KB, 4, 32).transpose(0, 2, 3, 1, 4).reshape(T, KB, 64, 32)
    packed = (c[..., 0::2] | (c[..., 1::2] << 4)).astype(np.uint8)
    s = np.zeros((T * 16, KB * 4), np.uint8)
    s[:m, : k // 32] = e8m0
    s = s.reshape(T, 16, KB, 4).transpose(0, 2, 3, 1).reshape(T, KB, 64)
    return packed.reshape(-1), s.reshape(-1)


def oracle_rows(x: np.ndarray):
    """Oracle mxfp4_quantize of each row of x [m, k]: codes [m, k], E8M0 [m, k/32], dequantized f64."""
    m, k = x.shape
    codes, s_block, e8, _, n = R.mxfp4_quantize(x.reshape(-1), 32)
    deq = R.mxfp4_dequantize(codes, s_block, (m, k), n).astype(np.float64)
    return codes.reshape(m, k), e8.reshape(m, k // 32), deq


def _values(shape, seed: int) -> np.ndarray:
    """Rows with magnitudes over many binades plus exact E2M1 midpoints and signed zeros."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(shape).astype(np.float32)
    x *= rng.choice(np.float32([1e-4, 0.02, 1.0, 20.0, 3000.0]), (shape[0], 1)).astype(np.float32)
    grid = np.float32([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0, -0.0, 0.0, -2.5, -6.0])
    k = min(shape[1], grid.size)
    x[0, :k] = grid[:k]
    return x


def _dev(a: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV).to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("m,k", [(1, 32), (17, 96), (40, 160), (64, 1024), (33, 4096)])
def test_mxfp4_quantize_tiled_bitexact(f4, m, k, dtype):
    print_case("mxfp4_quantize_tiled", f"m={m}", f"k={k}", f"dtype={dtype}")
    xg = _dev(_values((m, k), 100 + m), dtype)
    x = xg.float().cpu().numpy()  # the values the kernel sees
    codes, e8, _ = oracle_rows(x)
    xt_ref, xst_ref = tile_mx_np(codes, e8)
    q = f4.mxfp4_quantize_tiled(xg)
    torch.cuda.synchronize()
    xt = q.wt.cpu().numpy()
    xst = q.st.cpu().numpy()
    assert xt.shape == xt_ref.shape and xst.shape == xst_ref.shape
    assert np.array_equal(xt, xt_ref), f"codes differ at {np.flatnonzero(xt != xt_ref)[:8]}"
    assert np.array_equal(xst, xst_ref), f"scales differ at {np.flatnonzero(xst != xst_ref)[:8]}"


def test_mxfp4_quantize_tiled_matches_tile_of_quantize(f4):
    """Same bytes as the two-step path tile_fp4(mxfp4_quantize(x)) (both bit-exact on their own)."""
    print_case("mxfp4_quantize_tiled vs tile_fp4", "m=300", "k=640")
    g = torch.Generator(device="cpu").manual_seed(5)
    x = torch.randn(300, 640, generator=g).to(DEV, torch.bfloat16)
    a = f4.mxfp4_quantize_tiled(x)
    b = f4.tile_fp4(f4.mxfp4_quantize(x, 32))
    torch.cuda.synchronize()
    assert torch.equal(a.wt, b.wt) and torch.equal(a.st, b.st)


def _check_gemm(y: torch.Tensor, y_ref: np.ndarray, mag: np.ndarray, out_dtype: torch.dtype, what: str,
                k: int, splits: int = 1) -> None:
    """``splits`` K splits add one fp32 rounding each when their partials are summed."""
    yv = y.float().cpu().numpy().astype(np.float64)
    assert np.isfinite(yv).all(), f"{what}: non-finite output"
    err = np.abs(yv - y_ref)
    acc_bound = (k / 32 + 8 + splits) * 2.0**-24 * mag + 1e-30
    if out_dtype == torch.float32:
        worst = float((err / acc_bound).max())
        assert worst <= 1.0, f"{what}: fp32 output off by {worst:.2f}x the accumulation bound"
        return
    # half an ulp; fp16 also has subnormals down to 2**-24
    ulp_half = 2.0 ** (-8 if out_dtype == torch.bfloat16 else -11) * np.abs(y_ref)
    if out_dtype == torch.float16:
        ulp_half = ulp_half + 2.0**-25
    worst = float((err / (acc_bound + ulp_half + 1e-30)).max())
    assert worst <= 1.0, f"{what}: off by {worst:.2f}x the accumulation + rounding bound"
    scale = np.abs(y_ref).max()
    rel = float(err.max() / scale) if scale > 0 else float(err.max())
    rms = float(np.sqrt((y_ref**2).mean()))
    assert rel <= 1e-2, f"{what}: max-abs-rel {rel:.3e} > 1e-2"
    assert float((err / (2.0**-7 * (np.abs(y_ref) + rms) + 1e-30)).max()) <= 1.0, f"{what}: elementwise bound"


GEMM_SHAPES = [
    (1, 16, 32),  # one short k-block, one fragment row
    (5, 40, 96),  # partial 128-column block only
    (17, 300, 160),  # KB = 2 < stages - 1
    (256, 256, 384),  # exactly one tile, KB = 3
    (300, 520, 512),  # ragged m and n over several tiles, KB = 4 (steady state + tail)
    (64, 1000, 1056),  # KB = 9 with a 32-column last block
    (513, 257, 2048),  # m just past two tiles
    (1024, 2048, 1024),  # tile count a multiple of 8: XCD-grouped order
]


@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
def test_mxfp4_gemm_matches_oracle(f4, m, n, k):
    print_case("mxfp4_gemm", f"m={m}", f"n={n}", f"k={k}")
    x = _values((m, k), 7 + m)
    w = (np.random.default_rng(11 + n).standard_normal((n, k)) * 0.02).astype(np.float32)
    _, _, xd = oracle_rows(x)
    _, _, wd = oracle_rows(w)
    y_ref = xd @ wd.T
    mag = np.abs(xd) @ np.abs(wd).T
    xq = f4.mxfp4_quantize_tiled(_dev(x, torch.float32))
    tw = f4.tile_fp4(f4.mxfp4_quantize(_dev(w, torch.float32), 32))
    for out_dtype in (torch.float32, torch.bfloat16, torch.float16):
        if out_dtype == torch.float16 and np.abs(y_ref).max() > 6e4:
            continue
        y = f4.mxfp4_gemm(xq, tw, out_dtype=out_dtype)
        torch.cuda.synchronize()
        _check_gemm(y, y_ref, mag, out_dtype, f"mxfp4_gemm {m}x{n}x{k} {out_dtype}", k, splits=16)


SPLIT_SHAPES = [  # (m, n, k, splits): k-steps of 128 columns per split down to one, ragged last split
    (40, 300, 1024, 2),  # two splits of four k-steps
    (64, 1000, 1056, 3),  # KB = 9: splits of 3, the last with a 32-column block
    (17, 520, 2048, 4),  # KB = 16: 4+4+4+4 (5 would leave one empty: see the rejects test)
    (128, 512, 4096, 8),  # 8 splits of 4 steps
    (300, 260, 1024, 8),  # one k-step per split (shorter than the pipeline), ragged m and n
    (1, 64, 2048, 16),  # sixteen splits of one step, one row
]


@pytest.mark.parametrize("m,n,k,splits", SPLIT_SHAPES)
def test_mxfp4_gemm_split_k(f4, m, n, k, splits):
    """K split into fp32 partials summed in order: within the accumulation bound of the oracle
    product (one more rounding per split), deterministic, and equal to the one-pass result to fp32
    rounding."""
    from scratch_llm_amd import _lib

    print_case("mxfp4_gemm split-K", f"m={m}", f"n={n}", f"k={k}", f"splits={splits}")
    x = _values((m, k), 70 + m)
    w = (np.random.default_rng(3 + n).standard_normal((n, k)) * 0.02).astype(np.float32)
    _, _, xd = oracle_rows(x)
    _, _, wd = oracle_rows(w)
    b = np.random.default_rng(9).standard_normal(n).astype(np.float32)
    xq = f4.mxfp4_quantize_tiled(_dev(x, torch.float32))
    tw = f4.tile_fp4(f4.mxfp4_quantize(_dev(w, torch.float32), 32))
    lib = _lib.load()
    assert lib.sqx_mxfp4_gemm_workspace_bytes(m, n, k, splits) == splits * m * n * 4
    for out_dtype in (torch.float32, torch.bfloat16):
        bias = None if out_dtype == torch.float32 else _dev(b, torch.bfloat16)
        bb = np.zeros(n) if bias is None else R.round_bf16(b).astype(np.float64)
        y_ref = xd @ wd.T + bb[None, :]
        mag = np.abs(xd) @ np.abs(wd).T + np.abs(bb)[None, :]
        y = f4.mxfp4_gemm(xq, tw, bias, out_dtype=out_dtype, splits=splits)
        again = f4.mxfp4_gemm(xq, tw, bias, out_dtype=out_dtype, splits=splits)
        one = f4.mxfp4_gemm(xq, tw, bias, out_dtype=out_dtype, splits=1)
        torch.cuda.synchronize()
        _check_gemm(y, y_ref, mag, out_dtype, f"split {splits} {m}x{n}x{k} {out_dtype}", k, splits=splits)
        assert torch.equal(y, again), "split-K result not deterministic"
        if out_dtype == torch.float32:
            d = (y - one).abs().double().cpu().numpy()
            assert (d <= (2 * splits + 2) * 2.0**-24 * mag + 1e-30).all(), "split and one-pass differ beyond rounding"


def test_mxfp4_gemm_one_pass_entry_point(f4):
    """sqx_mxfp4_gemm (no workspace) is the one-split form of sqx_mxfp4_gemm_ws, bit for bit."""
    from scratch_llm_amd import _lib

    m, n, k = 96, 640, 2048
    print_case("mxfp4_gemm one-pass entry", f"m={m}", f"n={n}", f"k={k}")
    xq = f4.mxfp4_quantize_tiled(torch.randn(m, k, device=DEV))
    tw = f4.tile_fp4(f4.mxfp4_quantize(torch.randn(n, k, device=DEV) * 0.02, 32))
    bias = torch.randn(n, device=DEV, dtype=torch.bfloat16)
    y = torch.empty(m, n, device=DEV, dtype=torch.bfloat16)
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    assert lib.sqx_mxfp4_gemm(xq.wt.data_ptr(), xq.st.data_ptr(), tw.wt.data_ptr(), tw.st.data_ptr(), y.data_ptr(),
                              _lib.sqx_dtype(torch.bfloat16), bias.data_ptr(), m, n, k, st) == 0
    y1 = f4.mxfp4_gemm(xq, tw, bias, splits=1)
    torch.cuda.synchronize()
    assert torch.equal(y, y1)


def test_mxfp4_gemm_split_rejects(f4):
    from scratch_llm_amd import _lib

    m, n, k = 8, 64, 2048  # KB = 16
    xq = f4.mxfp4_quantize_tiled(torch.randn(m, k, device=DEV))
    tw = f4.tile_fp4(f4.mxfp4_quantize(torch.randn(n, k, device=DEV), 32))
    y = torch.empty(m, n, device=DEV, dtype=torch.bfloat16)
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    ws = torch.empty(lib.sqx_mxfp4_gemm_workspace_bytes(m, n, k, 4), device=DEV, dtype=torch.uint8)
    args = (xq.wt.data_ptr(), xq.st.data_ptr(), tw.wt.data_ptr(), tw.st.data_ptr(), y.data_ptr(),
            _lib.sqx_dtype(torch.bfloat16), None, m, n, k)
    assert lib.sqx_mxfp4_gemm_ws(*args, 5, ws.data_ptr(), ws.numel(), st) == -1  # 4+4+4+4+0: one empty
    assert "empty" in lib.sqx_last_error().decode()
    assert lib.sqx_mxfp4_gemm_ws(*args, 17, ws.data_ptr(), ws.numel(), st) == -1
    assert lib.sqx_mxfp4_gemm_ws(*args, 4, None, 0, st) == -1
    assert lib.sqx_mxfp4_gemm_ws(*args, 4, ws.data_ptr(), ws.numel() - 4, st) == -3  # SQX_E_SPACE
    assert lib.sqx_mxfp4_gemm_ws(*args, 4, ws.data_ptr() + 4, ws.numel() - 4, st) == -1  # alignment
    # automatic splitting without a workspace runs one pass
    assert lib.sqx_mxfp4_gemm_ws(*args, 0, None, 0, st) == 0
    y0 = y.clone()
    assert lib.sqx_mxfp4_gemm_ws(*args, 1, None, 0, st) == 0
    torch.cuda.synchronize()
    assert torch.equal(y, y0)


def test_mxfp4_gemm_bias(f4):
    m, n, k = 70, 300, 256
    print_case("mxfp4_gemm bias", f"m={m}", f"n={n}", f"k={k}")
    x = _values((m, k), 3)
    x[:, :] = np.clip(x, -50, 50)
    w = (np.random.default_rng(4).standard_normal((n, k)) * 0.02).astype(np.float32)
    b = np.random.default_rng(5).standard_normal(n).astype(np.float32)
    bb = R.round_bf16(b).astype(np.float64)
    _, _, xd = oracle_rows(x)
    _, _, wd = oracle_rows(w)
    y_ref = xd @ wd.T + bb[None, :]
    mag = np.abs(xd) @ np.abs(wd).T + np.abs(bb)[None, :]
    xq = f4.mxfp4_quantize_tiled(_dev(x, torch.float32))
    tw = f4.tile_fp4(f4.mxfp4_quantize(_dev(w, torch.float32), 32))
    y = f4.mxfp4_gemm(xq, tw, bias=_dev(b, torch.bfloat16), out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    _check_gemm(y, y_ref, mag, torch.bfloat16, "mxfp4_gemm bias", k)


@pytest.mark.parametrize("m", [1, 128, 200])
def test_mxfp4_linear_quantized_activations(f4, m):
    """The module-level API: F.linear(dequant(quant(x)), dequant(quant(W))) with bf16 activations."""
    n, k = 384, 1024
    print_case("mxfp4_linear quantize_activations", f"m={m}", f"n={n}", f"k={k}")
    g = torch.Generator(device="cpu").manual_seed(m)
    w = torch.randn(n, k, generator=g) * 0.02
    x = torch.randn(2, m, k, generator=g).to(torch.bfloat16)
    q = f4.mxfp4_quantize(w.to(DEV), 32)
    y = f4.mxfp4_linear(x.to(DEV), q, quantize_activations=True)
    torch.cuda.synchronize()
    assert y.shape == (2, m, n) and y.dtype == torch.bfloat16
    _, _, xd = oracle_rows(x.float().numpy().reshape(-1, k))
    _, _, wd = oracle_rows(w.numpy())
    y_ref = xd @ wd.T
    _check_gemm(y.reshape(-1, n), y_ref, np.abs(xd) @ np.abs(wd).T, torch.bfloat16, "mxfp4_linear act-quant", k)


@pytest.mark.parametrize("m", [4096, 128])
@pytest.mark.parametrize("n,k", [(28672, 8192), (8192, 28672)])
def test_mxfp4_gemm_config4_sampled(f4, n, k, m):
    """Config 4 at full size (M = 4096, and M = 128, where the k range is split automatically):
    weights ~N(0, 0.02), activations ~N(0, 1) bf16, both MXFP4; 24 rows x 160 columns of y against
    the oracle."""
    print_case("mxfp4_gemm config4", f"m={m}", f"n={n}", f"k={k}")
    g = torch.Generator(device=DEV).manual_seed(1000 + n)
    w = torch.randn(n, k, generator=g, device=DEV) * 0.02
    x = torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16)
    tw = f4.tile_fp4(f4.mxfp4_quantize(w, 32))
    xq = f4.mxfp4_quantize_tiled(x)
    y = f4.mxfp4_gemm(xq, tw)
    torch.cuda.synchronize()
    rng = np.random.default_rng(n)
    ri = np.sort(np.concatenate([[0, m - 1], rng.choice(m, 22, replace=False)]))
    ci = np.sort(np.concatenate([[0, n - 1], rng.choice(n, 158, replace=False)]))
    _, _, xd = oracle_rows(x[torch.from_numpy(ri).to(DEV)].float().cpu().numpy())
    _, _, wd = oracle_rows(w[torch.from_numpy(ci).to(DEV)].cpu().numpy())
    y_ref = xd @ wd.T
    ys = y[torch.from_numpy(ri).to(DEV)][:, torch.from_numpy(ci).to(DEV)]
    _check_gemm(ys, y_ref, np.abs(xd) @ np.abs(wd).T, torch.bfloat16, f"config4 {m}x{n}x{k}", k, splits=16)
    del w, x, tw, xq, y
    torch.cuda.empty_cache()


@pytest.mark.parametrize("m", [1, 8])
@pytest.mark.parametrize("n,k", [(28672, 8192), (8192, 28672)])
def test_mxfp4_act_linear_config4_small_m(f4, n, k, m):
    """Config 4's MXFP4-activation variant at M = 1 (and 8) on both Llama-3-70B MLP shapes: through
    ``mxfp4_linear(quantize_activations=True)`` (the FP4 GEMV on the dequantized rows) and through the
    fp4 MFMA GEMM, each against the product of the oracle's dequantized operands on 160 columns."""
    print_case("mxfp4 act-quant linear config4", f"m={m}", f"n={n}", f"k={k}")
    g = torch.Generator(device=DEV).manual_seed(2000 + n + m)
    w = torch.randn(n, k, generator=g, device=DEV) * 0.02
    x = torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16)
    q = f4.mxfp4_quantize(w, 32)
    y = f4.mxfp4_linear(x, q, quantize_activations=True)
    yg = f4.mxfp4_gemm(f4.mxfp4_quantize_tiled(x), f4.tile_fp4(q))
    torch.cuda.synchronize()
    assert y.shape == (m, n) and y.dtype == torch.bfloat16
    ci = np.sort(np.concatenate([[0, n - 1], np.random.default_rng(n + m).choice(n, 158, replace=False)]))
    _, _, xd = oracle_rows(x.float().cpu().numpy())
    _, _, wd = oracle_rows(w[torch.from_numpy(ci).to(DEV)].cpu().numpy())
    y_ref = xd @ wd.T
    mag = np.abs(xd) @ np.abs(wd).T
    cols = torch.from_numpy(ci).to(DEV)
    _check_gemm(y[:, cols], y_ref, mag, torch.bfloat16, f"act-quant GEMV {m}x{n}x{k}", k, splits=16)
    _check_gemm(yg[:, cols], y_ref, mag, torch.bfloat16, f"act-quant GEMM {m}x{n}x{k}", k, splits=16)
    del w, q, y, yg
    torch.cuda.empty_cache()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("shape", [(40, 1024), (1, 28672), (3, 1184)])
def test_mxfp4_fake_quant_rows_bitexact(f4, dtype, shape):
    """bf16(mxfp4_dequantize(mxfp4_quantize(row))) per row equals the oracle bit for bit, including
    all-zero blocks and values across many binades; one long row, and a grid whose last workgroup is
    partly past the blocks."""
    print_case("mxfp4 fake-quant rows", dtype, shape)
    x = _values(shape, 9 + shape[1])
    x[min(3, shape[0] - 1), :32] = 0.0
    xt = _dev(x, dtype)
    got = f4.mxfp4_fake_quant_rows(xt)
    _, _, xd = oracle_rows(xt.float().cpu().numpy())
    assert got.dtype == torch.bfloat16
    assert np.array_equal(got.float().cpu().numpy(), xd.astype(np.float32))


def test_mxfp4_fake_quant_rows_specials(f4):
    """Blocks holding NaN, +-inf or the largest float, each at a different lane of the eight that share
    a block (the block maximum joins the lanes' maxima). A block holding NaN has a NaN amax, so the
    reference's scale 2**ceil(log2(NaN)) is NaN and every dequantized value of the block is NaN (the
    oracle's integer exponent is undefined there); every other block equals the oracle bit for bit
    (an infinity's block decodes to signed zeros, the largest float's to 4 * 2**126 = inf)."""
    print_case("mxfp4 fake-quant rows specials")
    x = _values((2, 512), 5)
    fmax = np.finfo(np.float32).max
    for j, val in enumerate([np.nan, np.inf, -np.inf, fmax, -fmax, np.nan, np.inf, fmax]):
        x[0, 32 * j + 4 * j + 1] = val  # lane j of block j
    x[1, 32 * 3 + 30] = np.nan
    x[1, 32 * 5 + 2] = -np.inf
    xt = _dev(x, torch.float32)
    got = f4.mxfp4_fake_quant_rows(xt).float().cpu().numpy()
    nan_block = np.repeat(np.isnan(x.reshape(2, -1, 32)).any(axis=2), 32, axis=1)
    assert np.isnan(got[nan_block]).all()
    with np.errstate(invalid="ignore", over="ignore"):
        _, _, xd = oracle_rows(x)
    np.testing.assert_array_equal(got[~nan_block], xd.astype(np.float32)[~nan_block])


def test_mxfp4_gemm_rejects(f4):
    x = torch.randn(4, 64, device=DEV)
    xq = f4.mxfp4_quantize_tiled(x)
    w = f4.tile_fp4(f4.mxfp4_quantize(torch.randn(8, 96, device=DEV), 32))
    with pytest.raises(ValueError):
        f4.mxfp4_gemm(xq, w)
    with pytest.raises(ValueError):
        f4.mxfp4_quantize_tiled(torch.randn(4, 40, device=DEV))
    with pytest.raises(RuntimeError):
        f4.mxfp4_quantize_tiled(torch.randn(4, 64))
