"""Drop-in module plumbing on the CPU: which modules count as linears, the converters' skip rule,
the on-disk MXFP4 pair's refusals (k3/checkpoint.py:124-137, tests/test_k3_checkpoint.py:312-324),
and that a CPU module is refused rather than computed on the host."""

from __future__ import annotations

import pytest
import torch
from torch import nn

from scratch_llm_amd.quant import modules, nvfp4_mxfp4


class Linear(nn.Module):
    """Shaped like the reference's model.Linear (model.py:125-133): y = x @ W.T, no bias."""

    def __init__(self, i: int, o: int) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.randn(o, i) * 0.02)

    def forward(self, x):
        return x @ self.weight.T


class Block(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.wq = Linear(64, 64)
        self.proj = nn.Linear(64, 96)
        self.norm = nn.LayerNorm(64)


class Toy(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.embed = nn.Embedding(10, 64)
        self.blocks = nn.ModuleList([Block(), Block()])
        self.lm_head = nn.Linear(64, 10)


def test_is_linear():
    assert modules.is_linear(nn.Linear(4, 4))
    assert modules.is_linear(Linear(4, 4))
    assert not modules.is_linear(nn.LayerNorm(4))
    assert not modules.is_linear(nn.Embedding(4, 4))
    assert not modules.is_linear(Block())


def test_converter_skips_without_touching_the_device():
    """Every linear skipped: nothing is quantized, so nothing needs a GPU."""
    m = Toy()
    assert modules.convert_linears_to_int4(m, skip=("wq", "proj", "lm_head")) == []
    assert isinstance(m.blocks[0].proj, nn.Linear)


@pytest.mark.parametrize("conv,kw", [(modules.convert_linears_to_int4, {"group_size": 32}),
                                     (modules.convert_linears_to_int8, {}),
                                     (modules.convert_linears_to_mxfp4, {}), (modules.convert_linears_to_nvfp4, {})])
def test_cpu_weights_are_refused(conv, kw):
    with pytest.raises(RuntimeError):
        conv(Toy(), **kw)


def test_int4_layers_not_divisible_by_the_group_are_left_alone():
    m = Toy()
    assert modules.convert_linears_to_int4(m, group_size=128) == []  # in_features 64


@pytest.mark.parametrize(
    ("packed", "scale", "match"),
    [
        (torch.zeros(2, 16, dtype=torch.int8), torch.zeros(2, 1, dtype=torch.uint8), "uint8"),
        (torch.zeros(2, 16, dtype=torch.uint8), torch.zeros(1, 2, dtype=torch.uint8), "needs"),
        (torch.zeros(2, 8, dtype=torch.uint8), torch.zeros(2, 1, dtype=torch.uint8), "needs"),
        (torch.zeros(32, dtype=torch.uint8), torch.zeros(1, dtype=torch.uint8), r"\[out, in/2\]"),
        (torch.zeros(1, 16, dtype=torch.uint8), torch.full((1, 1), 0xFF, dtype=torch.uint8), "0xFF is NaN"),
    ],
    ids=["dtype", "scale-shape", "partial-group", "rank", "nan-scale"],
)
def test_mxfp4_pair_refusals(packed, scale, match):
    with pytest.raises(ValueError, match=match):
        modules.MXFP4Linear.from_packed(packed, scale)
    with pytest.raises(ValueError, match=match):
        nvfp4_mxfp4.dequantize_mxfp4(packed, scale)


def test_tensor_keyed_cache_replaces_on_in_place_update():
    """An in-place update rebuilds the derived value and replaces the entry: a weight updated twice
    still holds one cached value, and the entry goes when the weight is garbage-collected."""
    import gc

    from scratch_llm_amd.quant import _device

    cache = _device.TensorKeyedCache()
    q = torch.arange(12, dtype=torch.int8).reshape(3, 4)
    s = torch.ones(3, 1)
    builds = []

    def build():
        builds.append(int(q.sum()))
        return q.clone()

    v0 = cache.get((q, s), (128,), build)
    assert cache.get((q, s), (128,), build) is v0 and len(builds) == 1
    for step in (1, 2):
        q.add_(1)  # moves the version counter
        v = cache.get((q, s), (128,), build)
        assert torch.equal(v, q) and len(builds) == 1 + step
        assert len(cache) == 1
    assert cache.get((q, s), (64,), build) is not None and len(cache) == 2  # the extra key counts
    del q, v, v0
    gc.collect()
    assert len(cache) == 0
