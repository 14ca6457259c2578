"""Prefill dequant-GEMM parity on the MI355X (sqx_int4_gemm, sqx_fp4_gemm), taken by the tiled
linears from GEMM_MIN_M activation rows on.

The GEMM decodes every weight to exactly the reference's ``dequantize(...).to(x.dtype)`` value (INT4:
the fp32 ``(q - z) * s`` rounded to nearest even; MXFP4: ``e2m1 * 2**e``, exact), so the float64
product of x with those weights differs from the kernel only by fp32 accumulation, bounded by
``(k/32 + 8) * 2**-24 * sum_k |x_k w_k|`` (one rounded 32-term MFMA partial per step, two roundings
allowed per step), and the output rounding (half an ulp of the activation dtype). NVFP4 decodes
``e2m1 * s_block`` exactly and multiplies the fp32 sum by ``s_global``, so its weights differ from the
reference's ``(s_global * s_block * e2m1).to(x.dtype)`` by up to half an ulp: those cases use the
linear bar (max-abs-rel <= 1e-2, elementwise 2**-7 (|y| + rms y)).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import quant_ref as R
from tests.conftest import print_case

pytestmark = pytest.mark.gpu
DEV = "cuda"
ACT = {torch.bfloat16: "bf16", torch.float16: "f16"}


@pytest.fixture(scope="module")
def mods():
    from scratch_llm_amd import _lib
    from scratch_llm_amd.quant import awq, int4_group, nvfp4_mxfp4

    _lib.load()
    return int4_group, nvfp4_mxfp4, awq


def _check_exact_weights(y: torch.Tensor, x: np.ndarray, w: np.ndarray, bias: np.ndarray | None, dtype, what: str):
    """y against float64 x @ w.T (+ bias) with the accumulation + output-rounding bound."""
    k = x.shape[1]
    y_ref = x.astype(np.float64) @ w.astype(np.float64).T
    mag = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    if bias is not None:
        y_ref = y_ref + bias[None, :]
        mag = mag + np.abs(bias)[None, :]
    yv = y.float().cpu().numpy().astype(np.float64)
    assert np.isfinite(yv).all(), f"{what}: non-finite output"
    err = np.abs(yv - y_ref)
    ulp = 2.0 ** (-8 if dtype == torch.bfloat16 else -11) * np.abs(y_ref) + (2.0**-25 if dtype == torch.float16 else 0)
    if dtype == torch.float32:
        ulp = 0.0
    bound = (k / 32 + 8) * 2.0**-24 * mag + ulp + 1e-30
    worst = float((err / bound).max())
    assert worst <= 1.0, f"{what}: off by {worst:.2f}x the accumulation + rounding bound"


def _check_linear(y: torch.Tensor, y_ref: np.ndarray, what: str) -> None:
    yv = y.float().cpu().numpy().astype(np.float64)
    assert np.isfinite(yv).all(), f"{what}: non-finite output"
    err = np.abs(yv - y_ref)
    scale = np.abs(y_ref).max()
    rel = float(err.max() / scale) if scale > 0 else float(err.max())
    rms = float(np.sqrt((y_ref**2).mean()))
    assert rel <= 1e-2, f"{what}: max-abs-rel {rel:.3e} > 1e-2"
    assert float((err / (2.0**-7 * (np.abs(y_ref) + rms) + 1e-30)).max()) <= 1.0, f"{what}: elementwise bound"


def _inputs(m, n, k, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(n, k, generator=g) * 0.02
    x = torch.randn(m, k, generator=g)
    x[:, :: max(1, k // 40)] *= 20.0  # outlier channels
    return w, x.to(dtype)


INT4_CASES = [
    # m, n, k, group (the GEMM runs from 65 rows; fewer take the decode-regime kernels)
    (65, 16, 128, 128),
    (100, 40, 384, 64),
    (257, 300, 1024, 128),
    (300, 520, 1056, 32),  # 1056 = 8 blocks + 32 columns: partial last block
    (513, 257, 2048, 128),
    (1024, 1024, 4096, 128),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,n,k,group", INT4_CASES)
def test_int4_gemm_symmetric(mods, m, n, k, group, dtype):
    q4 = mods[0]
    print_case("int4 gemm sym", f"m={m}", f"n={n}", f"k={k}", f"group={group}", f"dtype={dtype}")
    w, x = _inputs(m, n, k, m + n + k, dtype)
    q, s = R.quantize_groupwise_int4(w.numpy(), group)
    w_eff = R.round_to(R.dequantize_groupwise_int4(q, s, group), ACT[dtype])
    tw = q4.tile_int4(torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV), None, group)
    bias = None
    if m % 2 == 1:
        bias = torch.randn(n, generator=torch.Generator().manual_seed(3)).to(dtype)
    y = q4.int4_linear_tiled(x.to(DEV), tw, None if bias is None else bias.to(DEV))
    torch.cuda.synchronize()
    assert y.shape == (m, n) and y.dtype == dtype
    b = None if bias is None else bias.float().numpy().astype(np.float64)
    _check_exact_weights(y, x.float().numpy(), w_eff, b, dtype, f"int4 gemm {m}x{n}x{k} g{group} {dtype}")


@pytest.mark.parametrize("param", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("m,n,k,group", [(65, 48, 256, 128), (300, 520, 1056, 32), (513, 257, 2048, 64)])
def test_int4_gemm_asymmetric(mods, m, n, k, group, param):
    q4 = mods[0]
    print_case("int4 gemm asym", f"m={m}", f"n={n}", f"k={k}", f"group={group}", f"param={param}")
    w, x = _inputs(m, n, k, 7 * m + n, torch.bfloat16)
    q, s, z = q4.quantize_groupwise_uint4_asym(w.to(DEV), group, param)
    w_eff = R.round_bf16(R.dequantize_groupwise_uint4_asym(q.cpu().numpy(), s.float().cpu().numpy(),
                                                           z.float().cpu().numpy(), group))
    tw = q4.tile_int4(q, s, z, group)
    y = q4.int4_linear_tiled(x.to(DEV), tw)
    torch.cuda.synchronize()
    _check_exact_weights(y, x.float().numpy(), w_eff, None, torch.bfloat16, f"int4 asym gemm {m}x{n}x{k}")


def test_int4_gemm_agrees_with_decode_kernel(mods):
    """Rows 64..: the GEMM and the streaming decode kernel (forced with k_slices) on the same inputs."""
    q4 = mods[0]
    m, n, k = 96, 384, 2048
    print_case("int4 gemm vs gemv", f"m={m}", f"n={n}", f"k={k}")
    w, x = _inputs(m, n, k, 5, torch.bfloat16)
    q, s = q4.quantize_groupwise_int4(w.to(DEV), 128)
    tw = q4.tile_int4(q, s, None, 128)
    xd = x.to(DEV)
    y_gemm = q4.int4_linear_tiled(xd, tw)
    y_gemv = q4.int4_linear_tiled(xd, tw, k_slices=4)
    torch.cuda.synchronize()
    _check_linear(y_gemm, y_gemv.double().cpu().numpy(), "gemm vs decode kernel")


@pytest.mark.parametrize("n,k", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)])
def test_awq_linear_config3_m2048(mods, n, k):
    """BASELINE config 3 at M = 2048 (the GEMM regime): 32 sampled rows against the oracle."""
    awq = mods[2]
    m = 2048
    print_case("awq gemm", f"n={n}", f"k={k}", f"m={m}")
    g = torch.Generator(device=DEV).manual_seed(n + k)
    w = torch.randn(n, k, generator=g, device=DEV) * 0.02
    s = torch.exp(torch.empty(k, device=DEV).uniform_(-0.6931, 0.6931, generator=g))
    quant = awq.quantize_awq_int4(w, chan_scale=s)
    x = torch.randn(m, k, generator=g, device=DEV)
    x[:, torch.randperm(k, generator=torch.Generator().manual_seed(k))[: k // 100].to(DEV)] *= 20.0
    x = x.to(torch.bfloat16)
    y = awq.awq_linear(x, quant)
    torch.cuda.synchronize()
    rows = torch.from_numpy(np.sort(np.random.default_rng(k).choice(m, 32, replace=False))).to(DEV)
    w_eff = R.round_bf16(awq.awq_dequantize(quant).cpu().numpy())
    y_ref = R.linear_f64(x[rows].float().cpu().numpy(), w_eff)
    # awq_linear multiplies x by 1/s (one bf16 rounding) before the GEMM: the AWQ bound of 2**-6
    yv = y[rows].float().cpu().numpy().astype(np.float64)
    err = np.abs(yv - y_ref)
    rms = float(np.sqrt((y_ref**2).mean()))
    assert float(err.max() / np.abs(y_ref).max()) <= 1e-2
    assert float((err / (2.0**-6 * (np.abs(y_ref) + rms))).max()) <= 1.0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,n,k", [(64, 16, 64), (128, 300, 1056), (257, 520, 4096), (1024, 1024, 8192)])
def test_mxfp4_gemm_bf16_activations(mods, m, n, k, dtype):
    f4 = mods[1]
    print_case("fp4 gemm mx", f"m={m}", f"n={n}", f"k={k}", f"dtype={dtype}")
    w, x = _inputs(m, n, k, 3 * m + k, dtype)
    codes, s_block, _, shape, nn = R.mxfp4_quantize(w.numpy(), 32)
    w_eff = R.round_to(R.mxfp4_dequantize(codes, s_block, shape, nn), ACT[dtype])
    q = f4.mxfp4_quantize(w.to(DEV), 32)
    y = f4.mxfp4_linear(x.to(DEV), q)
    torch.cuda.synchronize()
    _check_exact_weights(y, x.float().numpy(), w_eff, None, dtype, f"mxfp4 gemm {m}x{n}x{k} {dtype}")


@pytest.mark.parametrize("m,n,k", [(64, 48, 256), (300, 520, 1056), (513, 1024, 2048)])
def test_nvfp4_gemm(mods, m, n, k):
    """The kernel against the exact weights s_global * s_block * e2m1 (float64) with the
    accumulation bound (plus one rounding of the final s_global product), and against the
    reference's bf16-rounded weights with max-abs-rel <= 1e-2 and the bound those weights' own
    rounding implies: |y - y_ref| <= 2**-9 sum_k |x_k w_k| + the accumulation bound + half an ulp."""
    f4 = mods[1]
    print_case("fp4 gemm nv", f"m={m}", f"n={n}", f"k={k}")
    w, x = _inputs(m, n, k, m + 2 * n, torch.bfloat16)
    codes, sg, sb, shape, nn = R.nvfp4_quantize(w.numpy(), 16)
    w_exact = (R.e2m1_decode(codes).astype(np.float64) * (np.float64(sg) * sb.astype(np.float64))[:, None]).reshape(shape)
    w_ref = R.round_bf16(R.nvfp4_dequantize(codes, sg, sb, shape, nn))
    q = f4.nvfp4_quantize(w.to(DEV), 16)
    y = f4.nvfp4_linear(x.to(DEV), q)
    torch.cuda.synchronize()
    xf = x.float().numpy()
    _check_exact_weights(y, xf, w_exact, None, torch.bfloat16, f"nvfp4 gemm {m}x{n}x{k} (exact weights)")
    y_ref = R.linear_f64(xf, w_ref)
    yv = y.double().cpu().numpy()
    err = np.abs(yv - y_ref)
    assert float(err.max() / np.abs(y_ref).max()) <= 1e-2
    mag = np.abs(xf.astype(np.float64)) @ np.abs(w_exact).T
    bound = (2.0**-9 + (k / 32 + 8) * 2.0**-24) * mag + 2.0**-8 * np.abs(y_ref) + 1e-30
    assert float((err / bound).max()) <= 1.0, f"nvfp4 gemm {m}x{n}x{k} vs the reference's weights"


def test_fp4_gemm_fp32_activations(mods):
    """fp32 x runs as hi/lo bf16 rows through one GEMM pass with fp32 output (2m >= GEMM_MIN_M)."""
    f4 = mods[1]
    m, n, k = 80, 200, 512
    print_case("fp4 gemm fp32 x", f"m={m}", f"n={n}", f"k={k}")
    w, x = _inputs(m, n, k, 9, torch.float32)
    codes, s_block, _, shape, nn = R.mxfp4_quantize(w.numpy(), 32)
    w_eff = R.mxfp4_dequantize(codes, s_block, shape, nn).astype(np.float64)
    q = f4.mxfp4_quantize(w.to(DEV), 32)
    y = f4.mxfp4_linear(x.to(DEV), q)
    torch.cuda.synchronize()
    y_ref = x.double().numpy() @ w_eff.T
    rel = float(np.linalg.norm(y.double().cpu().numpy() - y_ref) / np.linalg.norm(y_ref))
    assert y.dtype == torch.float32 and rel < 1e-4, rel


def test_split_k_matches_unsplit(mods):
    """The k range split over workgroups (fp32 partials in the workspace, added in a fixed order) and
    the single pass (no workspace) agree to the accumulation bound; the split is deterministic."""
    q4 = mods[0]
    from scratch_llm_amd import _lib

    m, n, k = 64, 1024, 4096
    print_case("int4 gemm split-k", f"m={m}", f"n={n}", f"k={k}")
    lib = _lib.load()
    assert lib.sqx_gemm_workspace_bytes(m, n, k) > 0
    w, x = _inputs(m, n, k, 21, torch.bfloat16)
    q, s = q4.quantize_groupwise_int4(w.to(DEV), 128)
    tw = q4.tile_int4(q, s, None, 128)
    xd = x.to(DEV)

    def run(ws):
        y = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
        _lib.check(lib.sqx_int4_gemm(tw.wt.data_ptr(), tw.st.data_ptr(), None, _lib.DTYPE_F32, xd.data_ptr(),
                                     _lib.DTYPE_BF16, y.data_ptr(), None, m, n, k, 128, *_lib.ws_args(ws),
                                     _lib.stream_ptr(xd.device)), "split-k test")
        return y

    ws = _lib.gemm_workspace(m, n, k, xd.device)
    y_split, y_split2, y_one = run(ws), run(ws), run(None)
    torch.cuda.synchronize()
    assert torch.equal(y_split, y_split2)
    w_eff = R.round_bf16(R.dequantize_groupwise_int4(q.cpu().numpy(), s.cpu().numpy(), 128))
    for y in (y_split, y_one):
        _check_exact_weights(y, x.float().numpy(), w_eff, None, torch.bfloat16, "split-k")
