"""The second NVFP4 convention (the b_r6 rung: ceil-rounded UE4M3 block scales, E2M1 ties to even,
no global scale) on the MI355X against the oracle (oracle/nvfp4_ceil_ref.py, pinned in
tests/test_oracle_nvfp4_ceil.py).

Bit-exact: packed codes and scale codes for fp32 / bf16 / fp16 operands over eight decades of
magnitude (normal and subnormal scales), blocks whose quotients land exactly on every E2M1 midpoint,
zero blocks and negative values that round to zero; dequantize (fp32 and bf16); the elementwise
rules. Refusals: NaN / Inf and unrepresentable blocks raise ValueError, as in the reference.
GEMM: ``b_r6_gemm_packed`` against the float64 product of the two oracle-dequantized operands,
within the fp32 accumulation bound ``(K/32 + 8) * 2**-24 * sum_k |a_k b_k|`` (every product is exact).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import nvfp4_ceil_ref as C
from tests.conftest import print_case

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def nc():
    from scratch_llm_amd import _lib
    from scratch_llm_amd.quant import nvfp4_ceil

    _lib.load()
    return nvfp4_ceil


def _operand(rows, k, seed, dtype=torch.float32):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    x *= np.exp2(rng.uniform(-14, 8, (rows, 1))).astype(np.float32)  # per-row decades, some subnormal scales
    if rows >= 4 and k >= 32:
        x[0, :16] = 0.0  # zero block
        x[1, :16] = np.float32([6, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, -0.25, -0.75, -5.0, -2.5, 5.5, -5.5, 0.1, -0.2])
        x[2, 16:32] = x[1, :16] * 3.0  # the same ties at scale 3 (amax 18 -> scale ceil(3) = 3)
        x[3, :16] = np.float32([-6] + [-0.2] * 15)  # negatives rounding to zero
    return torch.from_numpy(x).to(dtype)


@pytest.mark.parametrize("rows,k,dtype", [(128, 64, torch.float32), (1000, 4096, torch.float32),
                                          (64, 256, torch.bfloat16), (33, 512, torch.float16), (7, 16, torch.float32)])
def test_quantize_dequantize_bitexact(nc, rows, k, dtype):
    print_case("nvfp4 ceil quantize", rows, k, dtype)
    x = _operand(rows, k, rows + k, dtype)
    op = nc.quantize_nvfp4(x.to(DEV))
    torch.cuda.synchronize()
    pr, sr = C.quantize(x.float().numpy())
    assert np.array_equal(op.scales.cpu().numpy(), sr)
    assert np.array_equal(op.packed.cpu().numpy(), pr)
    d32 = nc.dequantize_nvfp4(op)
    want = C.dequantize(pr, sr)
    assert np.array_equal(d32.cpu().numpy().view(np.uint32), want.view(np.uint32))
    d16 = nc.dequantize_nvfp4(op, torch.bfloat16)
    assert torch.equal(d16.float().cpu(), torch.from_numpy(want))  # every NVFP4 value is exact in bf16


def test_round_trip_and_idempotence_on_gpu(nc):
    x = (torch.randn(128, 64, generator=torch.Generator().manual_seed(1)) * 10.0).to(DEV)
    op = nc.quantize_nvfp4(x)
    dq = nc.dequantize_nvfp4(op)
    op2 = nc.quantize_nvfp4(dq)
    assert torch.equal(op.packed, op2.packed) and torch.equal(op.scales, op2.scales)
    sc = torch.from_numpy(C.ue4m3_value(op.scales.cpu().numpy())).to(DEV).repeat_interleave(16, dim=1)
    err = (x.double() - dq.double()).abs()
    assert bool((err <= 0.25 * torch.maximum(x.double().abs(), sc)).all())


def test_refusals(nc):
    for bad in (float("nan"), float("inf")):
        x = torch.zeros(64, 64, device=DEV)
        x[3, 7] = bad
        with pytest.raises(ValueError, match="NaN or Inf"):
            nc.quantize_nvfp4(x)
    big = torch.zeros(4, 32, device=DEV)
    big[2, 20] = 448.0 * 6.0 * 1.01
    with pytest.raises(ValueError, match="unrepresentable"):
        nc.quantize_nvfp4(big)
    with pytest.raises(ValueError, match="SF_VEC_SIZE"):
        nc.quantize_nvfp4(torch.zeros(4, 24, device=DEV))
    with pytest.raises(RuntimeError):
        nc.quantize_nvfp4(torch.zeros(4, 32))


def test_elementwise_rules(nc, known_answers):
    ka = known_answers["nvfp4_ceil"]
    ties = torch.tensor(ka["rne_ties"]["in"] + [-v for v in ka["rne_ties"]["in"]], dtype=torch.float64, device=DEV)
    assert np.array_equal(nc.e2m1_round_code(ties).cpu().numpy(), C.e2m1_round_code(ties.cpu().numpy()))
    rng = np.random.default_rng(5)
    v = np.concatenate([rng.uniform(0, 448, 20000), np.exp2(rng.uniform(-16, 8.8, 20000)), C._GRID,
                        np.nextafter(C._GRID[1:], 0), np.nextafter(C._GRID[:-1], 1000)])
    v = v[v <= 448]
    got = nc.ue4m3_ceil_code(torch.from_numpy(v).to(DEV)).cpu().numpy()
    assert np.array_equal(got, C.ue4m3_ceil_code(v))
    amax = torch.tensor([0.0] + ka["ceil_amaxes"], dtype=torch.float64, device=DEV)
    codes, scales = nc.scale_for_amax(amax)
    wc, ws = C.scale_for_amax(amax.cpu().numpy())
    assert np.array_equal(codes.cpu().numpy(), wc) and np.array_equal(scales.cpu().numpy(), ws)
    y = np.concatenate([rng.uniform(-7, 7, 20000), C._MIDS, -C._MIDS, np.nextafter(C._MIDS, 0), np.nextafter(C._MIDS, 9)])
    assert np.array_equal(nc.e2m1_round_code(torch.from_numpy(y).to(DEV)).cpu().numpy(), C.e2m1_round_code(y))
    with pytest.raises(ValueError, match="NanInfEncoding"):
        nc.e2m1_round_code(torch.tensor([float("inf")], device=DEV))
    with pytest.raises(ValueError, match="exceeds"):
        nc.ue4m3_ceil_code(torch.tensor([500.0], device=DEV))


def test_e2m1_sign_rules_code_bytes(nc, known_answers):
    """As code bytes: the scalar helper keeps the sign of negatives that round to zero (-0.2 -> 0x8,
    nvfp4_layout.py:402), the quantizer stores them as +0 (b_r6.py:217-223)."""
    ka = known_answers["nvfp4_ceil"]
    sc = ka["e2m1_scalar_codes"]
    got = nc.e2m1_round_code(torch.tensor(sc["in"], dtype=torch.float64, device=DEV)).cpu().tolist()
    assert got == sc["out"]
    qc = ka["e2m1_quantizer_codes"]
    vals = [v for v in qc["in"] if abs(v) > 1e-30 or v == 0.0]
    row = torch.zeros(1, 16, dtype=torch.float32)
    row[0, 0] = 6.0
    row[0, 1:1 + len(vals)] = torch.tensor(vals)
    op = nc.quantize_nvfp4(row.to(DEV))
    p = op.packed.cpu()
    codes = torch.stack((p & 0xF, p >> 4), dim=-1).reshape(-1).tolist()
    assert int(op.scales.item()) == 0x38
    assert codes == [7] + [qc["out"][qc["in"].index(v)] for v in vals] + [0] * (15 - len(vals))


def test_quantize_float64_operand(nc):
    """A float64 operand is quantized in float64, as the reference's ``x.to(float64)``: quotients one
    float64 ulp off an E2M1 midpoint (which fp32 would round onto it) take the side they lie on."""
    print_case("nvfp4 ceil quantize float64")
    rng = np.random.default_rng(11)
    x = rng.standard_normal((64, 256)) * np.exp2(rng.uniform(-10, 6, (64, 1)))
    mids = np.array(C._MIDS)
    for r in range(8):  # blocks of amax 6 (scale 1) whose entries sit just off every midpoint
        x[r, :16] = 0.0
        x[r, 0] = 6.0
        x[r, 1:8] = np.nextafter(mids, 10.0 if r % 2 else -10.0)
        x[r, 8:15] = -x[r, 1:8]
        x[r, 15] = 1e-300 if r < 4 else -1e-300
    xt = torch.from_numpy(x).to(DEV)
    op = nc.quantize_nvfp4(xt)
    pr, sr = C.quantize(x)
    assert np.array_equal(op.scales.cpu().numpy(), sr) and np.array_equal(op.packed.cpu().numpy(), pr)
    # the same operand read as fp32 would round those quotients onto the midpoints: different codes
    p32, _ = C.quantize(x.astype(np.float32))
    assert not np.array_equal(p32[:8], pr[:8])
    # integer operands are widened to float64 as well
    xi = torch.randint(-300, 300, (16, 64), dtype=torch.int32)
    opi = nc.quantize_nvfp4(xi.to(DEV))
    pi, si = C.quantize(xi.numpy().astype(np.float64))
    assert np.array_equal(opi.packed.cpu().numpy(), pi) and np.array_equal(opi.scales.cpu().numpy(), si)


@pytest.mark.parametrize("m,n,k", [(1, 256, 512), (64, 384, 1024), (200, 128, 4096), (8, 4096, 4096)])
def test_b_r6_gemm_against_dequantized_product(nc, m, n, k):
    print_case("b_r6 gemm", m, n, k)
    g = torch.Generator().manual_seed(m + n + k)
    a = torch.randn(m, k, generator=g)
    b = torch.randn(k, n, generator=g) * 0.1
    y = nc.b_r6_gemm(a.to(DEV), b.to(DEV))
    torch.cuda.synchronize()
    assert y.dtype == torch.float32 and y.shape == (m, n)
    qa = C.dequantize(*C.quantize(a.numpy())).astype(np.float64)
    qb = C.dequantize(*C.quantize(np.ascontiguousarray(b.numpy().T))).astype(np.float64)
    ref = qa @ qb.T
    assert np.array_equal(ref, C.reference_gemm(a.numpy(), b.numpy()))
    mag = np.abs(qa) @ np.abs(qb).T
    err = np.abs(y.cpu().numpy().astype(np.float64) - ref)
    worst = float((err / ((k / 32 + 8) * 2.0**-24 * mag + 1e-30)).max())
    assert worst <= 1.0, f"{worst:.2f}x the fp32 accumulation bound"
    assert torch.equal(nc.reference_gemm(a.to(DEV), b.to(DEV)), y)
    with pytest.raises(ValueError, match="disagree"):
        nc.b_r6_gemm(a.to(DEV), b[:-16].to(DEV))
