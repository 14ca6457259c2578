"""The decode-regime INT4 linear (1..64 activation rows, sqx_int4_skinny) on the MI355X against the
numpy oracle, with the bar of the other int4 linears (tests/test_gpu_int4.py): max-abs-rel 1e-2 of
the float64 product of x and the reference's bf16-cast dequantized weight, and the elementwise
bound 2**-7 * (|y_ref| + rms(y_ref)).

Every launch shape (tiles per workgroup, waves, K splits) is checked, on ragged shapes (rows not a
multiple of 16 or of the tiles per workgroup, columns not a multiple of 128, every group size,
asymmetric codes, fp16 activations, bias), together with determinism per shape and the refusals.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import quant_ref as R
from tests.conftest import print_case
from tests.test_gpu_int4 import _act, _check_linear, _weight

pytestmark = pytest.mark.gpu

DEV = "cuda"
E_ARG = -1  # SQX_E_ARG


@pytest.fixture(scope="module")
def q4():
    from scratch_llm_amd import _lib
    from scratch_llm_amd.quant import int4_group

    _lib.load()
    assert "libsqx_hip.so" in open("/proc/self/maps").read(), "native library not mapped"
    return int4_group


def _sym(q4, n, k, group, seed, std=0.05):
    w = _weight((n, k), seed, std=std).to(DEV)
    q, s = q4.quantize_groupwise_int4(w, group)
    w_eff = R.round_bf16(R.dequantize_groupwise_int4(q.cpu().numpy(), s.cpu().numpy(), group))
    return q4.tile_int4(q, s, None, group), w_eff


SHAPES = [  # (variant, tiles, waves, splits): 0 = waves splitting K, 1 = LDS-staged (4 or 8 compute waves)
    (0, 2, 1, 1), (0, 4, 1, 1), (0, 2, 8, 1), (0, 4, 8, 1), (0, 2, 3, 2), (0, 4, 4, 3), (0, 2, 8, 4), (0, 4, 2, 7),
    (1, 1, 4, 1), (1, 2, 4, 1), (1, 4, 4, 1), (1, 1, 4, 3), (1, 2, 4, 2), (1, 4, 4, 4),
    (1, 1, 8, 1), (1, 2, 8, 1), (1, 4, 8, 2), (1, 2, 8, 3),
]


@pytest.mark.parametrize("variant,tiles,waves,splits", SHAPES, ids=lambda v: str(v))
@pytest.mark.parametrize(
    "n,k,group,m",
    [
        (200, 1024, 128, 64),  # 13 tiles: the last workgroup holds one or three
        (48, 96, 32, 17),  # columns not a multiple of 128, three tiles
        (256, 1056, 32, 33),  # K tail with four groups per block
        (1000, 4096, 64, 16),
        (64, 512, 128, 9),
        (96, 2048, 128, 1),
    ],
)
def test_skinny_matches_oracle(q4, n, k, group, m, variant, tiles, waves, splits):
    print_case("skinny", n, k, group, m, variant, tiles, waves, splits)
    tw, w_eff = _sym(q4, n, k, group, n + k + m)
    x = _act(m, k, 3 * m + k).to(DEV)
    y = q4.int4_linear_skinny(x, tw, variant=variant, tiles=tiles, waves=waves, splits=splits)
    torch.cuda.synchronize()
    _check_linear(y, R.linear_f64(x.float().cpu().numpy(), w_eff), f"{k}->{n} g{group} M={m}")
    again = q4.int4_linear_skinny(x, tw, variant=variant, tiles=tiles, waves=waves, splits=splits)
    assert torch.equal(y, again)  # fixed-order sums


@pytest.mark.parametrize("m", [16, 17, 32, 64])
@pytest.mark.parametrize("n,k", [(6144, 4096), (28672, 4096), (4096, 14336), (1024, 4096)], ids=lambda v: str(v))
def test_skinny_llama_shapes_default(q4, n, k, m):
    """The library's launch shape for each row count, including four K splits on 64 tiles (1024)."""
    print_case("skinny llama", n, k, m)
    tw, w_eff = _sym(q4, n, k, 128, 7 * n + k, std=0.02)
    x = _act(m, k, m + 11).to(DEV)
    y = q4.int4_linear_skinny(x, tw)
    torch.cuda.synchronize()
    _check_linear(y, R.linear_f64(x.float().cpu().numpy(), w_eff), f"{k}->{n} M={m}")


@pytest.mark.parametrize(
    "n,k,group,m,waves,groups",
    [
        (4096, 4096, 128, 2, 0, 0), (4096, 4096, 128, 4, 0, 0), (4096, 4096, 128, 8, 0, 1), (4096, 4096, 128, 8, 0, 2),
        (4096, 4096, 128, 3, 4, 0), (1024, 4096, 128, 5, 8, 1), (1024, 4096, 128, 5, 8, 2), (6144, 4096, 128, 7, 16, 0),
        (4096, 14336, 128, 4, 0, 0), (4096, 14336, 128, 2, 16, 0), (4096, 14336, 128, 8, 0, 2),
        (4096, 14336, 128, 6, 16, 2),
        (1000, 1056, 32, 6, 0, 1), (1000, 1056, 32, 6, 0, 2),  # rows not a multiple of 16, a K tail, four groups a block
        (200, 96, 32, 3, 0, 0),  # columns not a multiple of 128, one block
        (200, 2048, 64, 7, 0, 2),  # 13 tiles: the two-group grid covers 16
        (48, 2048, 64, 8, 4, 1), (300, 4096, 32, 4, 4, 0),
    ],
)
def test_rows_gemv_matches_oracle(q4, n, k, group, m, waves, groups):
    """The multi-row GEMV (variant 2): 2..8 rows, the per-row activation sums charging the code offset;
    5..8 rows in one workgroup (groups 1) or as two workgroups of four rows per tile (groups 2)."""
    print_case("rows gemv", n, k, group, m, waves, groups)
    tw, w_eff = _sym(q4, n, k, group, 5 * n + k + m)
    x = _act(m, k, 7 * m + k).to(DEV)
    y = q4.int4_linear_skinny(x, tw, variant=2, waves=waves, tiles=groups)
    torch.cuda.synchronize()
    _check_linear(y, R.linear_f64(x.float().cpu().numpy(), w_eff),
                  f"rows {k}->{n} g{group} M={m} waves={waves} groups={groups}")
    assert torch.equal(y, q4.int4_linear_skinny(x, tw, variant=2, waves=waves, tiles=groups))  # fixed-order sums
    # each row alone through the one-row GEMV agrees to bf16 precision
    for r in (0, m - 1):
        y1 = q4.int4_linear_tiled(x[r:r + 1], tw)
        assert float((y1.float() - y[r:r + 1].float()).abs().max()) <= 2.0**-7 * float(y1.float().abs().max())


def test_rows_gemv_asymmetric_fp16_bias(q4):
    n, k = 400, 2048
    w = _weight((n, k), 23, dtype=torch.float32).numpy()
    for group, param in ((128, "bf16"), (64, "f32"), (32, "bf16")):
        qa, sa, za = R.quantize_groupwise_uint4_asym(w, group, param=param)
        pdt = torch.bfloat16 if param == "bf16" else torch.float32
        tw = q4.tile_int4(torch.from_numpy(qa).to(DEV), torch.from_numpy(sa).to(pdt).to(DEV),
                          torch.from_numpy(za).to(pdt).to(DEV), group)
        w_eff = R.dequantize_groupwise_uint4_asym(qa, sa, za, group)
        for dt, rnd in ((torch.bfloat16, "bf16"), (torch.float16, "f16")):
            for m in (2, 4, 8):
                print_case("rows gemv asym", group, param, dt, m)
                x = _act(m, k, group + m, dtype=dt).to(DEV)
                bias = torch.randn(n, dtype=dt, device=DEV)
                y = q4.int4_linear_skinny(x, tw, bias, variant=2)
                assert y.dtype == dt
                y_ref = R.linear_f64(x.float().cpu().numpy(), R.round_to(w_eff, rnd), bias.float().cpu().numpy())
                _check_linear(y, y_ref, f"rows asym g{group} {param} {dt} M={m}")


def test_skinny_asymmetric_fp16_bias(q4):
    n, k = 160, 1024
    w = _weight((n, k), 21, dtype=torch.float32).numpy()
    for group, param in ((128, "bf16"), (64, "f32"), (32, "bf16")):
        qa, sa, za = R.quantize_groupwise_uint4_asym(w, group, param=param)
        pdt = torch.bfloat16 if param == "bf16" else torch.float32
        tw = q4.tile_int4(torch.from_numpy(qa).to(DEV), torch.from_numpy(sa).to(pdt).to(DEV),
                          torch.from_numpy(za).to(pdt).to(DEV), group)
        w_eff = R.dequantize_groupwise_uint4_asym(qa, sa, za, group)
        for dt, rnd in ((torch.bfloat16, "bf16"), (torch.float16, "f16")):
            x = _act(40, k, group, dtype=dt).to(DEV)
            bias = torch.randn(n, dtype=dt, device=DEV)
            for variant, tiles, waves, splits in ((0, 2, 4, 1), (0, 4, 2, 2), (1, 1, 4, 1), (1, 4, 4, 2), (1, 2, 8, 1)):
                print_case("skinny asym", group, param, dt, variant, tiles, waves, splits)
                y = q4.int4_linear_skinny(x, tw, bias, variant=variant, tiles=tiles, waves=waves, splits=splits)
                assert y.dtype == dt
                y_ref = R.linear_f64(x.float().cpu().numpy(), R.round_to(w_eff, rnd), bias.float().cpu().numpy())
                _check_linear(y, y_ref, f"asym g{group} {param} {dt} {variant},{tiles},{waves},{splits}")


def test_skinny_zero_row_is_bias_and_shapes_agree(q4):
    n, k, m = 128, 2048, 24
    w = _weight((n, k), 5, std=0.02, dtype=torch.float32)
    w[9] = 0.0
    q, s = q4.quantize_groupwise_int4(w.to(DEV))
    tw = q4.tile_int4(q, s)
    x = _act(m, k, 6).to(DEV)
    bias = torch.randn(n, dtype=torch.bfloat16, device=DEV)
    outs = [q4.int4_linear_skinny(x, tw, bias, variant=v, tiles=r, waves=wv, splits=sp) for v, r, wv, sp in SHAPES]
    for y in outs:
        assert torch.equal(y[:, 9], bias[9].expand(m))
    ref = outs[0].float()
    for y in outs[1:]:  # different summation orders, the same value to bf16 precision
        assert float((y.float() - ref).abs().max()) <= 2.0**-7 * float(ref.abs().max())
    # the decode GEMV on the same weight agrees to the same precision
    y_gemv = q4.int4_linear_tiled(x, tw, bias, k_slices=4)
    assert float((y_gemv.float() - ref).abs().max()) <= 2.0**-7 * float(ref.abs().max())


def test_skinny_rejects(q4):
    from scratch_llm_amd import _lib

    tw, _ = _sym(q4, 64, 256, 128, 1)
    with pytest.raises(ValueError, match="at most 64 rows"):
        q4.int4_linear_skinny(torch.randn(65, 256, device=DEV, dtype=torch.bfloat16), tw)
    x = torch.randn(8, 256, device=DEV, dtype=torch.bfloat16)
    y = torch.empty(8, 64, device=DEV, dtype=torch.bfloat16)
    lib = _lib.load()
    args = (tw.wt.data_ptr(), tw.st.data_ptr(), None, _lib.sqx_dtype(tw.st.dtype), x.data_ptr(),
            _lib.sqx_dtype(x.dtype), y.data_ptr(), None, 8, 64, 256, 128)
    st = torch.cuda.current_stream().cuda_stream
    assert lib.sqx_int4_skinny(*args, 1, 3, 4, 1, None, 0, st) == E_ARG  # tiles 1, 2 or 4
    assert "bad launch shape" in lib.sqx_last_error().decode()
    assert lib.sqx_int4_skinny(*args, 0, 1, 2, 1, None, 0, st) == E_ARG  # waves splitting K: tiles 2 or 4
    assert lib.sqx_int4_skinny(*args, 0, 2, 9, 1, None, 0, st) == E_ARG  # waves <= 8
    assert lib.sqx_int4_skinny(*args, 1, 2, 6, 1, None, 0, st) == E_ARG  # LDS-staged: 4 or 8 compute waves
    assert lib.sqx_int4_skinny(*args, 3, 2, 4, 1, None, 0, st) == E_ARG  # no variant 3
    assert lib.sqx_int4_skinny(*args, 2, 0, 17, 1, None, 0, st) == E_ARG  # multi-row GEMV: at most 16 waves
    assert lib.sqx_int4_skinny(*args, 2, 3, 0, 1, None, 0, st) == E_ARG  # multi-row GEMV: 1 or 2 row groups
    assert lib.sqx_int4_skinny(*args, 2, 0, 0, 2, None, 0, st) == E_ARG  # multi-row GEMV: no K split
    assert lib.sqx_int4_skinny(*args, 0, 2, 1, 2, None, 0, st) == E_ARG  # splits need a workspace
    assert "workspace" in lib.sqx_last_error().decode()
    assert lib.sqx_int4_skinny_workspace_bytes(8, 64, 256, 2) == 2 * 8 * 64 * 4
    assert lib.sqx_int4_skinny_workspace_bytes(8, 64, 256, 1) == 0
    assert lib.sqx_int4_skinny(*args, 0, 2, 1, 1, None, 0, st) == 0
    assert lib.sqx_int4_skinny(*args, 1, 1, 8, 1, None, 0, st) == 0
    torch.cuda.synchronize()
