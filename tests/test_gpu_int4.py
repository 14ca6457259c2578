"""INT4 parity on the MI355X: the HIP kernels (through libsqx_hip.so) against the numpy oracle.

Bit-exact: quantize (codes and scales), pack, unpack, dequantize, tile layouts.
Linear: tolerance from the north star — max|y - y_ref| / max|y_ref| <= 1e-2, where y_ref is the
float64 product of x and the reference's bf16-cast dequantized weight — plus an elementwise bound
|y - y_ref| <= 2**-7 * (|y_ref| + rms(y_ref)) covering bf16 output rounding (2**-9) and the kernel
applying the fp32 group scale after accumulating exact code products (weight rounding 2**-9).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import quant_ref as R
from tests.conftest import print_case

pytestmark = pytest.mark.gpu

LLAMA_SHAPES = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]  # (out N, in K)
DEV = "cuda"


@pytest.fixture(scope="module")
def q4():
    from scratch_llm_amd import _lib
    from scratch_llm_amd.quant import int4_group

    _lib.load()
    maps = open("/proc/self/maps").read()
    assert "libsqx_hip.so" in maps, "native library not mapped"
    hips = {line.split()[-1] for line in maps.splitlines() if "libamdhip64" in line}
    assert len(hips) == 1, f"more than one HIP runtime mapped: {hips}"
    return int4_group


def _weight(shape, seed, std=0.02, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(dtype)


def _act(m, k, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(m, k, generator=g).to(dtype)


def _check_linear(y_gpu: torch.Tensor, y_ref: np.ndarray, what: str) -> float:
    y = y_gpu.float().cpu().numpy().astype(np.float64)
    assert np.isfinite(y).all(), f"{what}: non-finite output"
    err = np.abs(y - y_ref)
    scale = np.abs(y_ref).max()
    rel = float(err.max() / scale) if scale > 0 else float(err.max())
    rms = float(np.sqrt((y_ref**2).mean()))
    bound = 2.0**-7 * (np.abs(y_ref) + rms) + 1e-30
    worst = float((err / bound).max())
    assert rel <= 1e-2, f"{what}: max-abs-rel {rel:.3e} > 1e-2"
    assert worst <= 1.0, f"{what}: elementwise bound exceeded by {worst:.2f}x"
    return rel


# ------------------------------------------------------------------------------------------ bit-exact
@pytest.mark.parametrize(
    "shape,group,dtype",
    [
        ((64, 1024), 128, torch.float32),
        ((64, 1024), 128, torch.bfloat16),
        ((48, 512), 64, torch.float16),
        ((32, 256), 32, torch.float32),
        ((16, 1024), 512, torch.float32),
        ((16, 8), 8, torch.float32),
        ((8, 384), 96, torch.float32),  # generic (non power-of-two) group path
        ((4096, 4096), 128, torch.bfloat16),
    ],
)
def test_quantize_bitexact(q4, shape, group, dtype):
    print_case("quantize", shape, group, dtype)
    w = _weight(shape, 11, std=1.0, dtype=dtype)
    w[0, :group] = 0.0  # zero group -> FLT_MIN scale
    if shape[1] >= 2 * group:
        w[1, group : 2 * group] = torch.linspace(-7, 7, group).to(dtype)  # many exact ties
    q, s = q4.quantize_groupwise_int4(w.to(DEV), group)
    torch.cuda.synchronize()
    qr, sr = R.quantize_groupwise_int4(w.float().numpy(), group)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), sr.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), qr)


def test_quantize_ties_half_even(q4):
    w = torch.zeros(1, 128)
    w[0, :9] = torch.tensor([7.0, 2.5, -2.5, 3.5, 0.5, -0.5, 1.5, 6.5, -6.5])
    q, s = q4.quantize_groupwise_int4(w.to(DEV))
    assert s.item() == 1.0
    assert q[0, :9].cpu().tolist() == [7, 2, -2, 4, 0, 0, 2, 6, -6]


@pytest.mark.parametrize("n", [1, 2, 3, 5, 64, 255, 4097, 1 << 20])
def test_pack_unpack_bitexact(q4, n):
    print_case("pack", n)
    rng = np.random.default_rng(n)
    q = rng.integers(-8, 8, n).astype(np.int8)
    p = q4.pack_int4(torch.from_numpy(q).to(DEV))
    assert np.array_equal(p.cpu().numpy(), R.pack_int4(q))
    u = q4.unpack_int4(p, n)
    assert np.array_equal(u.cpu().numpy(), q)


def test_pack_known_answers(q4, known_answers):
    ka = known_answers["int4_pack"]
    p = q4.pack_int4(torch.tensor(ka["high_low_nibble"]["q"], dtype=torch.int8, device=DEV))
    assert p.cpu().tolist() == ka["high_low_nibble"]["packed"]
    alt = ka["alternating"]
    p = q4.pack_int4(torch.tensor(alt["q_pattern"] * alt["repeat"], dtype=torch.int8, device=DEV))
    assert p.cpu().tolist() == [alt["packed_byte"]] * alt["n_bytes"]
    m1 = ka["all_minus_one"]
    p = q4.pack_int4(torch.full((m1["n"],), m1["q_value"], dtype=torch.int8, device=DEV))
    assert p.cpu().tolist() == [m1["packed_byte"]] * m1["n_bytes"]
    with pytest.raises(ValueError, match="1-D"):
        q4.pack_int4(torch.zeros(2, 2, dtype=torch.int8, device=DEV))


def test_dequantize_exact(q4):
    w = _weight((96, 512), 5, std=1.0, dtype=torch.float32)
    q, s = q4.quantize_groupwise_int4(w.to(DEV))
    d = q4.dequantize_groupwise_int4(q, s)
    want = R.dequantize_groupwise_int4(q.cpu().numpy(), s.cpu().numpy())
    assert np.array_equal(d.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_tile_from_packed_matches_tile_from_codes(q4):
    w = _weight((100, 384), 6, std=1.0, dtype=torch.float32).to(DEV)
    q, s = q4.quantize_groupwise_int4(w, 64)
    a = q4.tile_int4(q, s, None, 64)
    b = q4.tile_int4_packed(q4.pack_int4(q.reshape(-1)), s, (100, 384), 64)
    assert torch.equal(a.wt, b.wt) and torch.equal(a.st, b.st)


# ------------------------------------------------------------------------------------------ linear
@pytest.fixture(scope="module", params=LLAMA_SHAPES, ids=lambda s: f"{s[1]}to{s[0]}")
def llama_weight(request, q4):
    n, k = request.param
    print_case("llama weight", n, k)
    w = _weight((n, k), 1000 + n + k)
    q, s = q4.quantize_groupwise_int4(w.to(DEV))
    qn, sn = q.cpu().numpy(), s.cpu().numpy()
    w_eff = R.round_bf16(R.dequantize_groupwise_int4(qn, sn))
    tw = q4.tile_int4(q, s)
    return n, k, q, s, tw, w_eff


@pytest.mark.parametrize("m", [1, 4, 8])
def test_linear_llama_shapes(q4, llama_weight, m):
    n, k, q, s, tw, w_eff = llama_weight
    print_case("linear", n, k, m)
    x = _act(m, k, 2000 + m)
    y = q4.int4_linear_tiled(x.to(DEV), tw)
    torch.cuda.synchronize()
    y_ref = R.linear_f64(x.float().numpy(), w_eff)
    _check_linear(y, y_ref, f"{k}->{n} M={m}")
    # the functional reference API (cached tiles) gives the identical result
    y2 = q4.w4a16_linear(x.to(DEV), q, s)
    assert torch.equal(y, y2)


@pytest.mark.parametrize("splits", [1, 2, 3, 8, 16])
def test_linear_kslice_counts_deterministic(q4, splits):
    n, k = 512, 4096
    w = _weight((n, k), 7).to(DEV)
    q, s = q4.quantize_groupwise_int4(w)
    tw = q4.tile_int4(q, s)
    x = _act(3, k, 8).to(DEV)
    y = q4.int4_linear_tiled(x, tw, k_slices=splits)
    y_again = q4.int4_linear_tiled(x, tw, k_slices=splits)
    assert torch.equal(y, y_again)  # fixed-order reduction of the wave partials
    w_eff = R.round_bf16(R.dequantize_groupwise_int4(q.cpu().numpy(), s.cpu().numpy()))
    _check_linear(y, R.linear_f64(x.float().cpu().numpy(), w_eff), f"splits={splits}")


@pytest.mark.parametrize(
    "n,k,group,m",
    [
        (1000, 1024, 128, 1),  # rows not a multiple of 16
        (40, 96, 32, 5),  # cols not a multiple of 128
        (64, 192, 64, 16),
        (48, 256, 128, 17),  # two MFMA row chunks
        (48, 256, 128, 64),  # four row chunks
        (48, 256, 128, 150),  # several passes of 64 rows
        (16, 128, 128, 1),
    ],
)
def test_linear_ragged_shapes(q4, n, k, group, m):
    print_case("ragged", n, k, group, m)
    w = _weight((n, k), n * k + m, std=0.05).to(DEV)
    q, s = q4.quantize_groupwise_int4(w, group)
    x = _act(m, k, m).to(DEV)
    y = q4.w4a16_linear(x, q, s, group_size=group)
    w_eff = R.round_bf16(R.dequantize_groupwise_int4(q.cpu().numpy(), s.cpu().numpy(), group))
    _check_linear(y, R.linear_f64(x.float().cpu().numpy(), w_eff), f"{k}->{n} g{group} M={m}")
    assert y.shape == (m, n) and y.dtype == torch.bfloat16


@pytest.mark.parametrize(
    "n,k,group,m",
    [
        (256, 768, 768, 3),  # group = in_features (the reference tests' per-row scale): 6 groups of 128
        (128, 4096, 4096, 1),  # one group per row at a Llama width, the one-row GEMV
        (96, 1024, 256, 8),
        (64, 288, 96, 2),  # 96 = 3 groups of 32
        (64, 320, 320, 64),  # 320 = 5 groups of 64, the row-tiled kernels
        (32, 512, 512, 100),  # the prefill GEMM
    ],
)
def test_linear_wide_groups(q4, n, k, group, m):
    """Groups wider than the kernels' 32 / 64 / 128 run as narrower groups with the scale repeated
    (int4_group.py:148-164 takes any group dividing in_features): the linear matches the oracle, and
    the tiles give back the reference's codes and one scale per source group."""
    print_case("wide group", n, k, group, m)
    w = _weight((n, k), n + k + group, std=0.05).to(DEV)
    q, s = q4.quantize_groupwise_int4(w, group)
    assert s.shape == (n, k // group)
    x = _act(m, k, m + 1).to(DEV)
    y = q4.w4a16_linear(x, q, s, group_size=group)
    w_eff = R.round_bf16(R.dequantize_groupwise_int4(q.cpu().numpy(), s.cpu().numpy(), group))
    _check_linear(y, R.linear_f64(x.float().cpu().numpy(), w_eff), f"{k}->{n} g{group} M={m}")
    tw = q4.tile_int4(q, s, None, group)
    assert tw.group_size == q4.tiled_group(group) and tw.param_repeat * tw.group_size == group
    qb, sb, _ = q4.untile_int4(tw)
    assert torch.equal(qb, q) and torch.equal(sb, s)
    tp = q4.tile_int4_packed(q4.pack_int4(q.reshape(-1)), s, (n, k), group)
    assert torch.equal(tp.wt, tw.wt) and torch.equal(tp.st, tw.st)
    with pytest.raises(ValueError, match="multiple of 32"):
        q4.w4a16_linear(x, q, s, group_size=48)


def test_wide_group_module_and_asymmetric(q4):
    from scratch_llm_amd.quant import modules

    print_case("wide group module")
    lin = torch.nn.Linear(1024, 200, bias=True).to(DEV)
    mod = modules.Int4Linear.from_linear(lin, group_size=512)
    q, s = q4.quantize_groupwise_int4(lin.weight.detach(), 512)
    assert torch.equal(mod.codes(), q) and torch.equal(mod.scales, s)
    assert torch.equal(mod.dequantized_weight(), q4.dequantize_groupwise_int4(q, s, 512))
    x = _act(5, 1024, 3).to(DEV)
    assert torch.equal(mod(x), q4.w4a16_linear(x, q, s, bias=lin.bias.detach(), group_size=512))
    # the build-defined asymmetric format with bf16 (scale, zero) pairs and 256-column groups
    w = _weight((64, 1024), 4, dtype=torch.float32).numpy()
    qa, sa, za = R.quantize_groupwise_uint4_asym(w, 256, param="bf16")
    tw = q4.tile_int4(torch.from_numpy(qa).to(DEV), torch.from_numpy(sa).to(torch.bfloat16).to(DEV),
                      torch.from_numpy(za).to(torch.bfloat16).to(DEV), 256)
    for m in (1, 8, 80):
        x = _act(m, 1024, 40 + m).to(DEV)
        y = q4.int4_linear_tiled(x, tw)
        w_eff = R.round_bf16(R.dequantize_groupwise_uint4_asym(qa, sa, za, 256))
        _check_linear(y, R.linear_f64(x.float().cpu().numpy(), w_eff), f"asym g256 M={m}")
    qb, sb, zb = q4.untile_int4(tw)
    assert np.array_equal(qb.cpu().numpy(), qa)
    assert torch.equal(sb.cpu(), torch.from_numpy(sa).to(torch.bfloat16))
    assert torch.equal(zb.cpu(), torch.from_numpy(za).to(torch.bfloat16))


def test_linear_zero_and_outlier_rows_bias_fp16(q4):
    n, k = 256, 1024
    w = _weight((n, k), 9, std=0.02, dtype=torch.float32)
    w[7] = 10.0  # outlier row (500x the rest; fp16 output stays finite)
    w[42] = 0.0  # zero row: output must be exactly the bias
    w = w.to(DEV)
    q, s = q4.quantize_groupwise_int4(w)
    x = _act(4, k, 10, dtype=torch.float16).to(DEV)
    bias = torch.randn(n, dtype=torch.float16, device=DEV)
    y = q4.w4a16_linear(x, q, s, bias=bias)
    assert y.dtype == torch.float16
    w_eff = R.round_to(R.dequantize_groupwise_int4(q.cpu().numpy(), s.cpu().numpy()), "f16")
    y_ref = R.linear_f64(x.float().cpu().numpy(), w_eff, bias.float().cpu().numpy())
    _check_linear(y[:, [i for i in range(n) if i != 7]], y_ref[:, [i for i in range(n) if i != 7]], "non-outlier rows")
    _check_linear(y[:, 7:8], y_ref[:, 7:8], "outlier row")
    assert torch.equal(y[:, 42], bias[42].expand(4))
    y0 = q4.w4a16_linear(x, q, s)
    assert torch.all(y0[:, 42] == 0)


def test_linear_asymmetric_bf16_params(q4):
    n, k = 1024, 4096
    w = _weight((n, k), 12, dtype=torch.float32).numpy()
    qa, sa, za = R.quantize_groupwise_uint4_asym(w, 128, param="bf16")
    tw = q4.tile_int4(
        torch.from_numpy(qa).to(DEV), torch.from_numpy(sa).to(torch.bfloat16).to(DEV),
        torch.from_numpy(za).to(torch.bfloat16).to(DEV), 128,
    )
    for m in (1, 8):
        x = _act(m, k, 30 + m).to(DEV)
        y = q4.int4_linear_tiled(x, tw)
        w_eff = R.round_bf16(R.dequantize_groupwise_uint4_asym(qa, sa, za))
        _check_linear(y, R.linear_f64(x.float().cpu().numpy(), w_eff), f"asym M={m}")


def test_linear_rejects_cpu_and_bad_shapes(q4):
    w = torch.randn(32, 256)
    with pytest.raises(RuntimeError, match="device tensors"):
        q4.quantize_groupwise_int4(w)
    with pytest.raises(ValueError, match="not divisible by group_size"):
        q4.quantize_groupwise_int4(torch.randn(32, 200, device=DEV))
    q, s = q4.quantize_groupwise_int4(w.to(DEV))
    with pytest.raises(ValueError):
        q4.int4_linear_tiled(torch.randn(2, 128, device=DEV, dtype=torch.bfloat16), q4.tile_int4(q, s))


def test_linear_back_to_back_shapes(q4):
    """Calls of different row-tile counts in sequence on one stream (regression: a former split-K
    design shared per-tile counters between calls) give results independent of their order."""
    outs = []
    for n, k, seed in ((512, 4096, 40), (4096, 4096, 41), (1024, 8192, 42), (512, 4096, 40)):
        print_case("back to back", n, k)
        w = _weight((n, k), seed).to(DEV)
        q, s = q4.quantize_groupwise_int4(w)
        x = _act(2, k, seed).to(DEV)
        y = q4.int4_linear_tiled(x, q4.tile_int4(q, s))
        w_eff = R.round_bf16(R.dequantize_groupwise_int4(q.cpu().numpy(), s.cpu().numpy()))
        _check_linear(y, R.linear_f64(x.float().cpu().numpy(), w_eff), f"{k}->{n}")
        outs.append(y)
    assert torch.equal(outs[0], outs[-1])
