"""Drop-in quantized linear modules and their converters, on the MI355X kernels.

The module pattern of the reference's ``Fp8Linear`` / ``convert_linears_to_fp8``
(src/scratch_llm/quant/fp8_weights.py:289-400) for the formats of this package: an ``nn.Module``
holding the quantized weight as buffers, ``from_linear``, ``dequantized_weight()`` (the fp32 weight
the kernel multiplies by) and ``forward``; ``convert_linears_to_<fmt>(root, skip=...)`` replaces
linears in place and returns the qualified names it replaced. Besides ``nn.Linear`` the converters
take the reference model's bias-free ``Linear`` (src/scratch_llm/model.py:125-133, ``y = x @ W.T``,
``weight [out, in]``), recognised by shape rather than type.

Every module computes on a ROCm device through libsqx_hip.so: a CPU tensor raises RuntimeError (the
reference's Fp8Linear keeps a CPU reference path; this package has none by design).
"""

from __future__ import annotations

import torch
from torch import Tensor, nn

from scratch_llm_amd import _lib
from scratch_llm_amd.quant import awq, int4_group, int8, nvfp4_mxfp4

__all__ = [
    "DEFAULT_SKIP",
    "AWQLinear",
    "Int4Linear",
    "Int8Linear",
    "MXFP4Linear",
    "NVFP4Linear",
    "convert_linears_to_awq",
    "convert_linears_to_int4",
    "convert_linears_to_int8",
    "convert_linears_to_mxfp4",
    "convert_linears_to_nvfp4",
    "is_linear",
]

#: Layers left unquantized by default (fp8_weights.py:361-364): the LM head, whose error lands on
#: the sampled token, and embeddings, which are a gather.
DEFAULT_SKIP = ("lm_head", "embed", "wte", "output")

def is_linear(m: nn.Module) -> bool:
    """``nn.Linear``, or a bias-free linear shaped like the reference's ``model.Linear``: a leaf module
    named ``Linear`` with a 2-D ``weight`` parameter and no ``bias`` (model.py:125-133)."""
    if isinstance(m, nn.Linear):
        return True
    w = getattr(m, "weight", None)
    return (
        type(m).__name__ == "Linear"
        and isinstance(w, torch.Tensor)
        and w.dim() == 2
        and getattr(m, "bias", None) is None
        and next(m.children(), None) is None
    )


def _weight_bias(m: nn.Module) -> tuple[Tensor, Tensor | None]:
    return m.weight.data, (None if getattr(m, "bias", None) is None else m.bias.data)


def _device_input(x: Tensor, *tensors: Tensor | None, fn: str) -> None:
    _lib.require_device(x, *tensors, fn=fn)


class _QuantLinear(nn.Module):
    in_features: int
    out_features: int

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, bias={self.bias is not None}"


class Int4Linear(_QuantLinear):
    """W4A16 with the reference's group-INT4 weight (int4_group.py:108-164). The module's state is the
    kernels' tiled copy only (buffers ``wt``, ``st``): the constructor takes the reference's tensors
    (``weight_packed``, the ``pack_int4`` bytes of the row-major codes, and fp32 ``scales``
    ``[out, in/g]``) and re-lays them once; ``weight_packed``, ``scales`` and ``codes()`` give them back
    bit for bit (``untile_int4``). ``forward`` is ``w4a16_linear`` on the tiles: the streaming decode
    kernel up to 64 rows, the prefill GEMM beyond."""

    wt: Tensor
    st: Tensor
    bias: Tensor | None

    def __init__(self, weight_packed: Tensor, scales: Tensor, bias: Tensor | None, in_features: int,
                 out_features: int, group_size: int = int4_group.GROUP_SIZE) -> None:
        super().__init__()
        int4_group._check_tiled_group(group_size)
        if in_features % group_size:
            raise ValueError(f"in_features={in_features} not divisible by group_size={group_size}")
        tw = int4_group.tile_int4_packed(weight_packed, scales, (out_features, in_features), group_size)
        self.register_buffer("wt", tw.wt)
        self.register_buffer("st", tw.st)
        self.register_buffer("bias", bias)
        self.in_features, self.out_features, self.group_size = in_features, out_features, group_size

    @classmethod
    def from_linear(cls, linear: nn.Module, *, group_size: int = int4_group.GROUP_SIZE) -> Int4Linear:
        w, b = _weight_bias(linear)
        q, s = int4_group.quantize_groupwise_int4(w, group_size)
        return cls(int4_group.pack_int4(q.reshape(-1)), s, None if b is None else b.clone(), w.shape[1], w.shape[0],
                   group_size)

    def tiled(self) -> int4_group.Int4Tiled:
        tg = int4_group.tiled_group(self.group_size)
        return int4_group.Int4Tiled(self.wt, self.st, None, self.out_features, self.in_features, tg,
                                    self.group_size // tg)

    def codes(self) -> Tensor:
        return int4_group.untile_int4(self.tiled())[0]

    @property
    def scales(self) -> Tensor:
        return int4_group.untile_int4(self.tiled())[1]

    @property
    def weight_packed(self) -> Tensor:
        return int4_group.pack_int4(self.codes().reshape(-1))

    def dequantized_weight(self) -> Tensor:
        """``(out, in)`` fp32 ``q * s`` (int4_group.py:132-142)."""
        q, s, _ = int4_group.untile_int4(self.tiled())
        return int4_group.dequantize_groupwise_int4(q, s, self.group_size)

    def forward(self, x: Tensor) -> Tensor:
        _device_input(x, self.wt, self.bias, fn="Int4Linear")
        return int4_group.int4_linear_tiled(x, self.tiled(), self.bias)


class AWQLinear(_QuantLinear):
    """W4A16 with an AWQ weight (awq.py:69-192): the group-INT4 codes of ``W * s`` and their group
    scales held as the kernels' tiled copy (buffers ``wt``, ``st``), and the per-input-channel
    ``chan_scale``; ``q``, ``group_scales`` and ``quant()`` give the reference's tensors back bit for bit.
    ``forward`` is ``awq_linear``."""

    wt: Tensor
    st: Tensor
    chan_scale: Tensor
    bias: Tensor | None

    def __init__(self, quant: awq.AWQQuant, bias: Tensor | None = None) -> None:
        super().__init__()
        tw = int4_group.tile_int4(quant.q, quant.group_scales, None, quant.group_size)
        self.register_buffer("wt", tw.wt)
        self.register_buffer("st", tw.st)
        self.register_buffer("chan_scale", quant.chan_scale)
        self.register_buffer("bias", bias)
        self.group_size = quant.group_size
        self.out_features, self.in_features = quant.q.shape

    @classmethod
    def from_linear(cls, linear: nn.Module, x: Tensor | None = None, chan_scale: Tensor | None = None, *,
                    group_size: int = awq.GROUP_SIZE, grid: int = 20) -> AWQLinear:
        w, b = _weight_bias(linear)
        quant = awq.quantize_awq_int4(w, x=x, chan_scale=chan_scale, group_size=group_size, grid=grid)
        return cls(quant, None if b is None else b.clone())

    def tiled(self) -> int4_group.Int4Tiled:
        tg = int4_group.tiled_group(self.group_size)
        return int4_group.Int4Tiled(self.wt, self.st, None, self.out_features, self.in_features, tg,
                                    self.group_size // tg)

    @property
    def q(self) -> Tensor:
        return int4_group.untile_int4(self.tiled())[0]

    @property
    def group_scales(self) -> Tensor:
        return int4_group.untile_int4(self.tiled())[1]

    def quant(self) -> awq.AWQQuant:
        q, gs, _ = int4_group.untile_int4(self.tiled())
        return awq.AWQQuant(q=q, group_scales=gs, chan_scale=self.chan_scale, group_size=self.group_size)

    def dequantized_weight(self) -> Tensor:
        return awq.awq_dequantize(self.quant())

    def forward(self, x: Tensor) -> Tensor:
        _device_input(x, self.wt, self.bias, fn="AWQLinear")
        return awq.awq_linear_tiled(x, self.tiled(), self.chan_scale, self.bias)


class Int8Linear(_QuantLinear):
    """Weight-only int8: per-output-channel symmetric codes of
    ``quantize_symmetric(W.float(), axis=0)`` (int8.py:102-125) held as the kernels' tiled copy (buffer
    ``wt``) with the fp32 ``scale [out, 1]``; ``q`` gives the codes back bit for bit. ``forward`` is
    ``F.linear(x, (q * s).to(x.dtype), bias)`` without materialising the weight."""

    wt: Tensor
    scale: Tensor
    bias: Tensor | None

    def __init__(self, q: Tensor, scale: Tensor, bias: Tensor | None = None) -> None:
        super().__init__()
        self.out_features, self.in_features = q.shape
        tw = int8.tile_int8(q, scale)
        self.register_buffer("wt", tw.wt)
        self.register_buffer("scale", tw.scale.reshape(-1, 1))
        self.register_buffer("bias", bias)

    @classmethod
    def from_linear(cls, linear: nn.Module) -> Int8Linear:
        w, b = _weight_bias(linear)
        q, s = int8.quantize_symmetric(w.float(), axis=0)
        return cls(q, s, None if b is None else b.clone())

    def tiled(self) -> int8.Int8Tiled:
        return int8.Int8Tiled(self.wt, self.scale.reshape(-1), self.out_features, self.in_features)

    @property
    def q(self) -> Tensor:
        return int8.untile_int8(self.tiled())

    def dequantized_weight(self) -> Tensor:
        return int8.dequantize_symmetric(self.q, self.scale)

    def forward(self, x: Tensor) -> Tensor:
        _device_input(x, self.wt, self.bias, fn="Int8Linear")
        return int8.int8_linear_tiled(x, self.tiled(), self.bias)


class MXFP4Linear(_QuantLinear):
    """MXFP4 weight in the on-disk compressed-tensors form (k3/checkpoint.py:92-144): the constructor
    takes ``weight_packed`` uint8 ``[out, in/2]`` and E8M0 ``weight_scale`` uint8 ``[out, in/32]`` and
    holds only their tiled copy (buffers ``wt``, ``st``: a byte permutation, no repack on the host);
    ``weight_packed`` / ``weight_scale`` give the pair back bit for bit. ``forward`` is
    ``F.linear(x, mxfp4_dequantize(W).to(x.dtype))``; with ``quantize_activations``
    the rows of ``x`` are MXFP4-quantized too and the product runs on the block-scaled fp4 MFMA."""

    wt: Tensor
    st: Tensor
    bias: Tensor | None

    def __init__(self, weight_packed: Tensor, weight_scale: Tensor, bias: Tensor | None = None, *,
                 quantize_activations: bool = False) -> None:
        super().__init__()
        rows, cols = nvfp4_mxfp4._check_mxfp4_pair(weight_packed, weight_scale)
        tw = nvfp4_mxfp4.tile_mxfp4_packed(weight_packed, weight_scale)
        self.register_buffer("wt", tw.wt)
        self.register_buffer("st", tw.st)
        self.register_buffer("bias", bias)
        self.out_features, self.in_features = rows, cols
        self.quantize_activations = quantize_activations

    @classmethod
    def from_linear(cls, linear: nn.Module, *, quantize_activations: bool = False) -> MXFP4Linear:
        w, b = _weight_bias(linear)
        packed, e8 = nvfp4_mxfp4.mxfp4_pack_weight(nvfp4_mxfp4.mxfp4_quantize(w, nvfp4_mxfp4.MXFP4_GROUP))
        return cls(packed, e8, None if b is None else b.clone(), quantize_activations=quantize_activations)

    @classmethod
    def from_packed(cls, weight_packed: Tensor, weight_scale: Tensor, bias: Tensor | None = None, *,
                    quantize_activations: bool = False) -> MXFP4Linear:
        """Load one checkpoint tensor pair straight into the kernel layout (refusing what the
        reference loader refuses: non-uint8 halves, bad shapes, the NaN scale 0xFF)."""
        return cls(weight_packed, weight_scale, bias, quantize_activations=quantize_activations)

    def tiled(self) -> nvfp4_mxfp4.FP4Tiled:
        return nvfp4_mxfp4.FP4Tiled(self.wt, self.st, _lib.FP4_MX, None, self.out_features, self.in_features)

    @property
    def weight_packed(self) -> Tensor:
        return nvfp4_mxfp4.untile_fp4(self.tiled())[0]

    @property
    def weight_scale(self) -> Tensor:
        return nvfp4_mxfp4.untile_fp4(self.tiled())[1]

    def dequantized_weight(self) -> Tensor:
        return nvfp4_mxfp4.dequantize_mxfp4(*nvfp4_mxfp4.untile_fp4(self.tiled()))

    def forward(self, x: Tensor) -> Tensor:
        _device_input(x, self.wt, self.bias, fn="MXFP4Linear")
        tw = self.tiled()
        if not self.quantize_activations:
            return nvfp4_mxfp4.fp4_linear_tiled(x, tw, self.bias)
        *batch, k = x.shape
        xq = nvfp4_mxfp4.mxfp4_quantize_tiled(x.reshape(-1, k))
        return nvfp4_mxfp4.mxfp4_gemm(xq, tw, self.bias, x.dtype).reshape(*batch, tw.rows)


class NVFP4Linear(_QuantLinear):
    """NVFP4 weight (nvfp4_mxfp4.py:190-231), held as the kernels' tiled copy (buffers ``wt``, ``st``:
    the E2M1 codes and the E4M3 bytes of the block scales) with the fp32 ``s_global``; ``tensor()``
    gives the reference's ``NVFP4Tensor`` back bit for bit. ``forward`` is
    ``F.linear(x, nvfp4_dequantize(W).to(x.dtype))``."""

    wt: Tensor
    st: Tensor
    s_global: Tensor
    bias: Tensor | None

    def __init__(self, q: nvfp4_mxfp4.NVFP4Tensor, bias: Tensor | None = None) -> None:
        super().__init__()
        if len(q.shape) != 2:
            raise ValueError(f"a linear needs a 2-D weight, got shape {tuple(q.shape)}")
        tw = nvfp4_mxfp4.tile_fp4(q)
        self.register_buffer("wt", tw.wt)
        self.register_buffer("st", tw.st)
        self.register_buffer("s_global", tw.s_global)
        self.register_buffer("bias", bias)
        self.block = q.block
        self.out_features, self.in_features = int(q.shape[0]), int(q.shape[1])

    @classmethod
    def from_linear(cls, linear: nn.Module, *, block: int = 16) -> NVFP4Linear:
        w, b = _weight_bias(linear)
        return cls(nvfp4_mxfp4.nvfp4_quantize(w, block), None if b is None else b.clone())

    def tiled(self) -> nvfp4_mxfp4.FP4Tiled:
        return nvfp4_mxfp4.FP4Tiled(self.wt, self.st, _lib.FP4_NV, self.s_global, self.out_features, self.in_features)

    def tensor(self) -> nvfp4_mxfp4.NVFP4Tensor:
        packed, e4 = nvfp4_mxfp4.untile_fp4(self.tiled())
        n = self.out_features * self.in_features
        codes = nvfp4_mxfp4.unpack_fp4(packed.reshape(-1), n).reshape(-1, self.block)
        # one E4M3 byte per 16 columns; a block of `block` columns repeats its scale
        s_block = nvfp4_mxfp4.e4m3_values(e4[:, :: self.block // 16].reshape(-1))
        return nvfp4_mxfp4.NVFP4Tensor(codes, self.s_global, s_block,
                                       torch.Size((self.out_features, self.in_features)), n, self.block)

    def dequantized_weight(self) -> Tensor:
        return nvfp4_mxfp4.nvfp4_dequantize(self.tensor())

    def forward(self, x: Tensor) -> Tensor:
        _device_input(x, self.wt, self.bias, fn="NVFP4Linear")
        return nvfp4_mxfp4.fp4_linear_tiled(x, self.tiled(), self.bias)


# --------------------------------------------------------------------------------------------------
# Converters (fp8_weights.py:367-400)
# --------------------------------------------------------------------------------------------------
def _convert(root: nn.Module, make, accept, skip: tuple[str, ...]) -> list[str]:
    """Replace, in place, every linear child whose (local) name contains no ``skip`` entry and that
    ``accept`` takes; returns the qualified names replaced. As in the reference converter, ``skip``
    is matched against each child's own attribute name."""
    replaced: list[str] = []
    for name, child in list(root.named_children()):
        if is_linear(child):
            if any(s in name for s in skip) or not accept(child):
                continue
            setattr(root, name, make(child))
            replaced.append(name)
        else:
            replaced.extend(f"{name}.{sub}" for sub in _convert(child, make, accept, skip))
    return replaced


def _in_features(m: nn.Module) -> int:
    return int(m.weight.shape[1])


def convert_linears_to_int4(root: nn.Module, *, skip: tuple[str, ...] = DEFAULT_SKIP,
                            group_size: int = int4_group.GROUP_SIZE) -> list[str]:
    """Replace every linear under ``root`` with :class:`Int4Linear` (layers whose ``in_features`` is
    not a multiple of ``group_size`` are left alone)."""
    return _convert(root, lambda m: Int4Linear.from_linear(m, group_size=group_size),
                    lambda m: _in_features(m) % group_size == 0, skip)


def convert_linears_to_awq(root: nn.Module, chan_scales: dict[str, Tensor] | None = None, *,
                           calib: dict[str, Tensor] | None = None, skip: tuple[str, ...] = DEFAULT_SKIP,
                           group_size: int = awq.GROUP_SIZE, grid: int = 20) -> list[str]:
    """Replace every linear under ``root`` with :class:`AWQLinear`. The scale of a layer comes from
    ``chan_scales`` (keyed by the layer's local name) or is searched on its calibration activations
    ``calib[name]``; a layer with neither is left alone."""
    chan_scales, calib = chan_scales or {}, calib or {}
    names: dict[int, str] = {}

    def accept(m: nn.Module) -> bool:
        return _in_features(m) % group_size == 0 and id(m) in names

    def make(m: nn.Module) -> AWQLinear:
        key = names[id(m)]
        return AWQLinear.from_linear(m, x=calib.get(key), chan_scale=chan_scales.get(key), group_size=group_size,
                                     grid=grid)

    for name, mod in root.named_modules():
        local = name.rsplit(".", 1)[-1]
        if is_linear(mod) and (local in chan_scales or local in calib):
            names[id(mod)] = local
    return _convert(root, make, accept, skip)


def convert_linears_to_int8(root: nn.Module, *, skip: tuple[str, ...] = DEFAULT_SKIP) -> list[str]:
    """Replace every linear under ``root`` with :class:`Int8Linear`."""
    return _convert(root, Int8Linear.from_linear, lambda m: True, skip)


def convert_linears_to_mxfp4(root: nn.Module, *, skip: tuple[str, ...] = DEFAULT_SKIP,
                             quantize_activations: bool = False) -> list[str]:
    """Replace every linear under ``root`` with :class:`MXFP4Linear` (``in_features % 32 == 0``)."""
    return _convert(root, lambda m: MXFP4Linear.from_linear(m, quantize_activations=quantize_activations),
                    lambda m: _in_features(m) % nvfp4_mxfp4.MXFP4_GROUP == 0, skip)


def convert_linears_to_nvfp4(root: nn.Module, *, skip: tuple[str, ...] = DEFAULT_SKIP, block: int = 16) -> list[str]:
    """Replace every linear under ``root`` with :class:`NVFP4Linear` (``in_features % block == 0``)."""
    return _convert(root, lambda m: NVFP4Linear.from_linear(m, block=block),
                    lambda m: _in_features(m) % block == 0, skip)
