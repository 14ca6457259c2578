"""Drop-in modules on the MI355X: conversion of a model holding both nn.Linear and the reference's
bias-free model.Linear shape, each module's forward against F.linear with its own
``dequantized_weight()`` cast to the activation dtype (the reference composition), and the on-disk
MXFP4 pair loaded straight into the kernel layout against the oracle restatement of
k3/checkpoint.py:92-144 and the reference's named byte values (tests/test_k3_checkpoint.py:281-292).

Tolerance: max-abs-rel <= 1e-2 (the north star's linear bar) and, elementwise, the bound the
reference composition's own roundings imply: its bf16 weights are within 2**-9 of the dequantized
weight (|dy| <= 2**-9 sum_k |x_k w_k|), fp32 accumulation adds at most (k/32 + 8) 2**-24 sum_k |x_k w_k|
and the bf16 output half an ulp (2**-8 |y| allowed). AWQ rounds x / s to bf16 once more (another
2**-9 sum_k |x_k w_k|)."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

from oracle import quant_ref as R
from tests.conftest import print_case

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def mods():
    from scratch_llm_amd import _lib
    from scratch_llm_amd.quant import modules

    _lib.load()
    return modules


class Linear(nn.Module):
    """Shaped like the reference's model.Linear (model.py:125-133)."""

    def __init__(self, i: int, o: int) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.randn(o, i) * 0.02)

    def forward(self, x):
        return x @ self.weight.T


class Block(nn.Module):
    def __init__(self, d: int, f: int) -> None:
        super().__init__()
        self.wq = Linear(d, d)
        self.up = nn.Linear(d, f)
        self.down = nn.Linear(f, d, bias=False)


class Toy(nn.Module):
    def __init__(self, d: int = 256, f: int = 512) -> None:
        super().__init__()
        self.embed = nn.Embedding(32, d)
        self.blocks = nn.ModuleList([Block(d, f), Block(d, f)])
        self.lm_head = nn.Linear(d, 32)


EXPECTED = ["blocks.0.wq", "blocks.0.up", "blocks.0.down", "blocks.1.wq", "blocks.1.up", "blocks.1.down"]


def _check(y: torch.Tensor, x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None, what: str,
           weight_terms: int = 1) -> None:
    """y against F.linear(x, w.to(bf16), bias) in float64 (x, w the values the reference multiplies)."""
    x64 = x.double().cpu()
    w64 = w.double().cpu()
    y_ref = x64 @ w.to(torch.bfloat16).double().cpu().T
    if bias is not None:
        y_ref = y_ref + bias.double().cpu()
    mag = x64.abs() @ w64.abs().T
    k = x.shape[-1]
    yv = y.double().cpu()
    assert torch.isfinite(yv).all(), what
    err = (yv - y_ref).abs()
    rel = float(err.max() / y_ref.abs().max())
    assert rel <= 1e-2, f"{what}: max-abs-rel {rel:.3e}"
    bound = (weight_terms * 2.0**-9 + (k / 32 + 8) * 2.0**-24) * mag + 2.0**-8 * y_ref.abs() + 1e-30
    assert float((err / bound).max()) <= 1.0, f"{what}: elementwise bound {float((err / bound).max()):.2f}x"


@pytest.mark.parametrize("fmt", ["int4", "int8", "mxfp4", "mxfp4_act", "nvfp4"])
@pytest.mark.parametrize("m", [1, 5, 96])
def test_convert_and_forward(mods, fmt, m):
    print_case("modules", fmt, f"m={m}")
    torch.manual_seed(7)
    model = Toy().to(DEV)
    conv = {
        "int4": lambda r: mods.convert_linears_to_int4(r),
        "int8": lambda r: mods.convert_linears_to_int8(r),
        "mxfp4": lambda r: mods.convert_linears_to_mxfp4(r),
        "mxfp4_act": lambda r: mods.convert_linears_to_mxfp4(r, quantize_activations=True),
        "nvfp4": lambda r: mods.convert_linears_to_nvfp4(r),
    }[fmt]
    assert conv(model) == EXPECTED
    assert isinstance(model.lm_head, nn.Linear)
    x = torch.randn(m, 256, device=DEV).to(torch.bfloat16)
    for name in EXPECTED:
        mod = model.get_submodule(name)
        xin = x if mod.in_features == 256 else torch.randn(m, mod.in_features, device=DEV).to(torch.bfloat16)
        y = mod(xin)
        torch.cuda.synchronize()
        assert y.shape == (m, mod.out_features) and y.dtype == torch.bfloat16
        xr = xin
        if fmt == "mxfp4_act":  # the reference composition also dequantizes the MXFP4-quantized activations
            from scratch_llm_amd.quant import nvfp4_mxfp4 as f4

            xr = f4.mxfp4_dequantize(f4.mxfp4_quantize(xin, 32)).to(torch.bfloat16)
        _check(y, xr, mod.dequantized_weight(), mod.bias, f"{fmt} {name} m={m}")


def test_awq_module(mods):
    print_case("awq module")
    torch.manual_seed(3)
    model = Toy().to(DEV)
    scales = {"wq": torch.exp(torch.empty(256, device=DEV).uniform_(-0.69, 0.69)),
              "up": torch.exp(torch.empty(256, device=DEV).uniform_(-0.69, 0.69))}
    calib = {"down": torch.randn(64, 512, device=DEV)}
    names = mods.convert_linears_to_awq(model, scales, calib=calib)
    assert names == EXPECTED
    for name in EXPECTED:
        mod = model.get_submodule(name)
        x = torch.randn(9, mod.in_features, device=DEV).to(torch.bfloat16)
        y = mod(x)
        _check(y, x, mod.dequantized_weight(), mod.bias, f"awq {name}", weight_terms=2)


def test_mxfp4_pair_loads_straight_into_the_kernel(mods):
    """Every byte against every scale code (the pattern of tests/test_k3_checkpoint.py:260-277):
    dequantized_weight() equals the oracle's k3 decode exactly, and the linear runs on the pair."""
    from scratch_llm_amd.quant import nvfp4_mxfp4 as f4

    n = 253  # scale codes 0..252: 6 * 2**(252 - 127) stays finite in fp32 and bf16
    packed = torch.arange(256, dtype=torch.uint8).repeat(n, 1)
    scale = ((torch.arange(n)[:, None] + torch.arange(16)[None, :]) % n).to(torch.uint8)
    want = R.dequantize_mxfp4_checkpoint(packed.numpy(), scale.numpy())
    mod = mods.MXFP4Linear.from_packed(packed.to(DEV), scale.to(DEV))
    got = mod.dequantized_weight()
    torch.cuda.synchronize()
    assert got.dtype == torch.float32 and got.shape == (n, 512)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want.astype(np.float32).view(np.uint32))
    # the named values: 0x80 = (+0, -0), 0x7F = (-6, +6), 0x21 = (1/2, 1); scale 0 is 2**-127
    p = torch.zeros(3, 16, dtype=torch.uint8)
    p[:, :3] = torch.tensor([0x80, 0x7F, 0x21], dtype=torch.uint8)
    sc = torch.tensor([[127], [0], [252]], dtype=torch.uint8)
    w = f4.dequantize_mxfp4(p.to(DEV), sc.to(DEV)).cpu()
    assert w[0, :6].tolist() == [0.0, -0.0, -6.0, 6.0, 0.5, 1.0]
    assert not w[0, 0].signbit() and w[0, 1].signbit()
    assert w[1, 4].item() == 2.0**-128 and w[1, 3].item() == 6 * 2.0**-127
    with pytest.raises(ValueError, match="not exact"):
        f4.dequantize_mxfp4(torch.full((1, 16), 0x07, dtype=torch.uint8, device=DEV),
                            torch.full((1, 1), 254, dtype=torch.uint8, device=DEV))
    # float64 holds every value of every E8M0 code exactly (k3/checkpoint.py:136-144): scale byte 254
    # with the largest codes (6 * 2**127 = 1.5 * 2**129) and every other code, against the oracle
    big = f4.dequantize_mxfp4(torch.full((1, 16), 0xF7, dtype=torch.uint8, device=DEV),
                              torch.full((1, 1), 254, dtype=torch.uint8, device=DEV), dtype=torch.float64).cpu()
    assert big.dtype == torch.float64 and big[0, :2].tolist() == [6 * 2.0**127, -6 * 2.0**127]
    rng = np.random.default_rng(3)
    pk = rng.integers(0, 256, (255, 64), dtype=np.uint8)
    e8 = np.repeat(np.arange(255, dtype=np.uint8)[:, None], 4, axis=1)  # every finite code, one per row
    e8[::7, 1] = 0
    got = f4.dequantize_mxfp4(torch.from_numpy(pk).to(DEV), torch.from_numpy(e8).to(DEV), dtype=torch.float64).cpu()
    want = R.dequantize_mxfp4_checkpoint(pk, e8)
    assert np.array_equal(got.numpy().view(np.uint64), want.view(np.uint64))
    # a linear on realistic scales: the pair of a quantized N(0, 0.02) weight
    wt = torch.randn(384, 1024, device=DEV) * 0.02
    q = f4.mxfp4_quantize(wt, 32)
    pk, e8 = f4.mxfp4_pack_weight(q)
    lin = mods.MXFP4Linear.from_packed(pk, e8)
    assert torch.equal(lin.dequantized_weight(), f4.mxfp4_dequantize(q))
    x = torch.randn(7, 1024, device=DEV).to(torch.bfloat16)
    _check(lin(x), x, f4.mxfp4_dequantize(q), None, "pair")


def test_modules_refuse_cpu_input(mods):
    model = Toy().to(DEV)
    mods.convert_linears_to_int8(model)
    with pytest.raises(RuntimeError):
        model.blocks[0].up(torch.randn(2, 256))


@pytest.mark.parametrize("rows,cols,group,kind,pdt", [(100, 384, 128, 0, torch.float32), (33, 96, 32, 1, torch.bfloat16),
                                                      (16, 4096, 64, 1, torch.float32), (257, 1056, 32, 0, torch.float32)])
def test_untile_int4_round_trip(mods, rows, cols, group, kind, pdt):
    """untile_int4(tile_int4(q, s[, z])) gives q, s (and z) back bit for bit, ragged rows and columns
    (padding rows and columns of the tiles are skipped)."""
    from scratch_llm_amd.quant import int4_group as i4

    print_case("untile int4", rows, cols, group, kind, pdt)
    g = torch.Generator().manual_seed(rows * cols)
    lo, hi = (-8, 8) if kind == 0 else (0, 16)
    q = torch.randint(lo, hi, (rows, cols), generator=g, dtype=torch.int8).to(DEV)
    s = torch.rand(rows, cols // group, generator=g).to(pdt).to(DEV)
    z = None if kind == 0 else torch.randint(0, 16, (rows, cols // group), generator=g).to(pdt).to(DEV)
    tw = i4.tile_int4(q, s, z, group)
    q2, s2, z2 = i4.untile_int4(tw)
    assert torch.equal(q2, q) and torch.equal(s2, s)
    assert (z2 is None) if z is None else torch.equal(z2, z)


@pytest.mark.parametrize("rows,cols", [(100, 200), (16, 64), (1000, 4096)])
def test_untile_int8_round_trip(mods, rows, cols):
    from scratch_llm_amd.quant import int8 as q8

    print_case("untile int8", rows, cols)
    q = torch.randint(-128, 128, (rows, cols), generator=torch.Generator().manual_seed(cols), dtype=torch.int8).to(DEV)
    tw = q8.tile_int8(q, torch.ones(rows, device=DEV))
    assert torch.equal(q8.untile_int8(tw), q)


@pytest.mark.parametrize("rows,cols,nv", [(100, 96, False), (33, 4096, False), (64, 160, True), (5, 8192, True)])
def test_untile_fp4_round_trip(mods, rows, cols, nv):
    """untile_fp4 of a tiled pair gives the reference's packed bytes and scale bytes back, bit for bit."""
    from scratch_llm_amd import _lib
    from scratch_llm_amd.quant import nvfp4_mxfp4 as f4

    print_case("untile fp4", rows, cols, nv)
    g = torch.Generator().manual_seed(rows + cols)
    packed = torch.randint(0, 256, (rows, cols // 2), generator=g, dtype=torch.uint8).to(DEV)
    bs = 16 if nv else 32
    if nv:
        vals = f4.e4m3_values(torch.randint(0, 0x7F, (rows, cols // bs), generator=g, dtype=torch.uint8).to(DEV))
        lib = _lib.load()
        wt = torch.empty(lib.sqx_fp4_tiled_weight_bytes(rows, cols), dtype=torch.uint8, device=DEV)
        st = torch.empty(lib.sqx_fp4_tiled_scale_bytes(rows, cols, _lib.FP4_NV), dtype=torch.uint8, device=DEV)
        _lib.check(lib.sqx_fp4_tile(packed.data_ptr(), 1, vals.data_ptr(), _lib.FP4_SCALE_NV_F32, bs, rows, cols,
                                    wt.data_ptr(), st.data_ptr(), _lib.stream_ptr(packed.device)), "tile")
        tw = f4.FP4Tiled(wt, st, _lib.FP4_NV, torch.ones((), device=DEV), rows, cols)
        p2, s2 = f4.untile_fp4(tw)
        assert torch.equal(p2, packed) and torch.equal(f4.e4m3_values(s2), vals)
    else:
        e8 = torch.randint(100, 150, (rows, cols // bs), generator=g, dtype=torch.uint8).to(DEV)
        p2, s2 = f4.untile_fp4(f4.tile_mxfp4_packed(packed, e8))
        assert torch.equal(p2, packed) and torch.equal(s2, e8)


def test_modules_hold_only_the_tiled_copy(mods):
    """Every module's buffers are the tiled weight (plus its per-row / global scales, the AWQ channel
    scale and the bias): no full-size copy in the reference's format stays beside it, and the
    reference's tensors come back exactly from the tiles."""
    from scratch_llm_amd.quant import int4_group as i4

    lin = nn.Linear(1024, 512).to(DEV)
    for name, make in [("int4", mods.Int4Linear.from_linear), ("int8", mods.Int8Linear.from_linear),
                       ("mxfp4", mods.MXFP4Linear.from_linear), ("nvfp4", mods.NVFP4Linear.from_linear)]:
        mod = make(lin)
        names = {n for n, _ in mod.named_buffers()}
        assert "wt" in names and not names & {"weight_packed", "q", "codes", "weight_scale"}, (name, names)
        weight_bytes = sum(b.numel() * b.element_size() for n, b in mod.named_buffers() if n not in ("bias",))
        per_weight = weight_bytes / (1024 * 512)
        assert per_weight <= {"int4": 0.54, "int8": 1.01, "mxfp4": 0.54, "nvfp4": 0.57}[name], (name, per_weight)
    mod = mods.Int4Linear.from_linear(lin)
    q, s = i4.quantize_groupwise_int4(lin.weight.data)
    assert torch.equal(mod.codes(), q) and torch.equal(mod.scales, s)
    assert torch.equal(mod.weight_packed, i4.pack_int4(q.reshape(-1)))
    awq_mod = mods.AWQLinear.from_linear(lin, chan_scale=torch.linspace(0.5, 2.0, 1024, device=DEV))
    names = {n for n, _ in awq_mod.named_buffers()}
    assert names == {"wt", "st", "chan_scale", "bias"}
    qa = awq_mod.quant()
    assert qa.q.dtype == torch.int8 and tuple(qa.q.shape) == (512, 1024)
