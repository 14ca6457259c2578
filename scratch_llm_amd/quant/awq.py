"""AWQ (activation-aware weight quantization) on MI355X — the API of ``scratch_llm.quant.awq``.

Same names, signatures, defaults, dataclasses (``AWQQuant``, ``AWQSearchResult``) and ``ValueError``
messages as ``src/scratch_llm/quant/awq.py`` (cited per function), on ROCm device tensors:

* ``quantize_awq_int4`` with a channel scale quantizes ``W * s`` in one HIP kernel, bit-identical
  to the reference's codes and group scales;
* ``awq_dequantize`` is bit-identical;
* ``awq_linear`` runs the int4 linear on ``x / s`` (``(x/s) @ (W s)^T = x @ W^T``, awq.py:15-16), so
  the weight is never materialised; it agrees with the reference within the bf16 tolerance;
* ``search_awq_scale`` runs the reference's grid search. The activation scale, the channel scale at
  each grid point and the fake-quantized weight come from HIP kernels; the fp32 calibration
  products ``x @ W^T`` are plain library GEMMs. ``act_scale`` sums in fp64, not in torch's order,
  so the chosen alpha at near-ties is not pinned bit-for-bit.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor

from scratch_llm_amd import _lib
from scratch_llm_amd.quant import _device
from scratch_llm_amd.quant.int4_group import (  # noqa: F401  (module attributes, as in the reference)
    GROUP_SIZE,
    TILED_GROUPS,
    Int4Tiled,
    dequantize_groupwise_int4,
    int4_linear_tiled,
    int4_linear_tiled_f32,
    mse,
    quantize_groupwise_int4,
    tile_int4,
    tiled_group,
)

__all__ = [
    "AWQQuant",
    "AWQSearchResult",
    "act_scale",
    "awq_dequantize",
    "awq_linear",
    "quantize_awq_int4",
    "search_awq_scale",
]


@dataclass(frozen=True)
class AWQQuant:
    """An AWQ-quantized W4A16 weight (awq.py:69-82): group-int4 codes ``q`` and ``group_scales`` of
    ``W * chan_scale``, the per-input-channel scale ``chan_scale`` ``[in]`` and the group size."""

    q: Tensor
    group_scales: Tensor
    chan_scale: Tensor
    group_size: int


@dataclass(frozen=True)
class AWQSearchResult:
    """The chosen scale, its grid exponent and the calibration MSE (awq.py:85-91)."""

    chan_scale: Tensor
    ratio: float
    calib_mse: float


def _stream(t: Tensor) -> int:
    return _lib.stream_ptr(t.device)


def act_scale(x: Tensor) -> Tensor:
    """Per-input-channel mean absolute activation ``E[|x_j|]``, fp32 ``[in]`` (awq.py:94-101)."""
    _lib.require_device(x, fn="act_scale")
    k = x.shape[-1]
    x2 = x.reshape(-1, k)
    if x2.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        x2 = x2.to(torch.float32)
    x2 = x2.contiguous()
    out = torch.empty(k, dtype=torch.float32, device=x2.device)
    with torch.cuda.device(x2.device):
        _lib.check(_lib.load().sqx_col_absmean(x2.data_ptr(), _lib.sqx_dtype(x2.dtype), x2.shape[0], k, out.data_ptr(),
                                               _stream(x2)), "act_scale")
    return out


def _grid_scale(a: Tensor, ratio: float) -> Tensor:
    """``_normalize_scale(a ** ratio)`` (awq.py:104-112, 141-142) on the device."""
    out = torch.empty_like(a)
    with torch.cuda.device(a.device):
        _lib.check(_lib.load().sqx_awq_scale(a.data_ptr(), a.numel(), float(ratio), out.data_ptr(), _stream(a)),
                   "search_awq_scale")
    return out


def _awq_dequant_weight(w: Tensor, chan_scale: Tensor, group_size: int) -> Tensor:
    """Quantize ``W * s`` to group-INT4, dequantize and fold ``1/s`` back (awq.py:115-119)."""
    rows, cols = w.shape
    if cols % group_size != 0:
        raise ValueError(f"in_features={cols} not divisible by group_size={group_size}")
    wc = w.contiguous() if w.dtype in (torch.float32, torch.bfloat16, torch.float16) else w.float().contiguous()
    s = chan_scale.to(torch.float32).contiguous()
    out = torch.empty(rows, cols, dtype=torch.float32, device=w.device)
    with torch.cuda.device(w.device):
        _lib.check(_lib.load().sqx_awq_fake_quant(wc.data_ptr(), _lib.sqx_dtype(wc.dtype), s.data_ptr(), rows, cols,
                                                  group_size, out.data_ptr(), _stream(wc)), "_awq_dequant_weight")
    return out


def search_awq_scale(w: Tensor, x: Tensor, group_size: int = GROUP_SIZE, grid: int = 20) -> AWQSearchResult:
    """Grid-search ``s = act_scale(x) ** alpha`` minimizing the layer-output MSE (awq.py:122-151):
    for ``alpha = i/grid``, ``i`` in ``[0, grid]``, quantize ``W * s``, fold ``1/s`` back and compare
    ``x @ W_eff^T`` with the fp32 ``x @ W^T``. ``alpha = 0`` is naive INT4."""
    if w.dim() != 2:
        raise ValueError(f"expected a 2-D weight, got shape {tuple(w.shape)}")
    _lib.require_device(w, x, fn="search_awq_scale")
    wf = w.to(torch.float32)
    xf = x.to(torch.float32)
    y_ref = xf @ wf.t()
    a = act_scale(xf)
    best: AWQSearchResult | None = None
    for i in range(grid + 1):
        ratio = i / grid
        s = _grid_scale(a, ratio)
        w_eff = _awq_dequant_weight(wf, s, group_size)
        cur = mse(y_ref, xf @ w_eff.t())
        if best is None or cur < best.calib_mse:
            best = AWQSearchResult(chan_scale=s, ratio=ratio, calib_mse=cur)
    assert best is not None
    return best


def quantize_awq_int4(
    w: Tensor,
    x: Tensor | None = None,
    chan_scale: Tensor | None = None,
    group_size: int = GROUP_SIZE,
    grid: int = 20,
) -> AWQQuant:
    """AWQ-quantize a weight ``[out, in]`` to W4A16 (awq.py:154-175): pass calibration activations
    ``x`` to search the scale, or a precomputed ``chan_scale`` ``[in]``. The codes are the group-INT4
    quantization of ``W * s``."""
    if chan_scale is not None:
        scale = chan_scale.to(torch.float32)
    elif x is not None:
        scale = search_awq_scale(w, x, group_size=group_size, grid=grid).chan_scale
    else:
        raise ValueError("provide either calibration activations `x` or a `chan_scale`")
    if w.dim() != 2:
        raise ValueError(f"expected a 2-D weight, got shape {tuple(w.shape)}")
    rows, cols = w.shape
    if cols % group_size != 0:
        raise ValueError(f"in_features={cols} not divisible by group_size={group_size}")
    _lib.require_device(w, scale, fn="quantize_awq_int4")
    wc = w.contiguous() if w.dtype in (torch.float32, torch.bfloat16, torch.float16) else w.float().contiguous()
    sc = scale.contiguous()
    q = torch.empty(rows, cols, dtype=torch.int8, device=w.device)
    gs = torch.empty(rows, cols // group_size, dtype=torch.float32, device=w.device)
    with torch.cuda.device(w.device):
        _lib.check(_lib.load().sqx_awq_quantize(wc.data_ptr(), _lib.sqx_dtype(wc.dtype), sc.data_ptr(), rows, cols,
                                                group_size, q.data_ptr(), gs.data_ptr(), _stream(wc)),
                   "quantize_awq_int4")
    return AWQQuant(q=q, group_scales=gs, chan_scale=scale, group_size=group_size)


def awq_dequantize(quant: AWQQuant) -> Tensor:
    """The effective fp32 weight ``dequant(q, group_scales) / chan_scale`` (awq.py:178-181)."""
    q, gs, s = quant.q, quant.group_scales, quant.chan_scale
    _lib.require_device(q, gs, s, fn="awq_dequantize")
    rows, cols = q.shape
    qc = q.to(torch.int8).contiguous()
    gsc = gs.to(torch.float32).contiguous()
    sc = s.to(torch.float32).contiguous()
    out = torch.empty(rows, cols, dtype=torch.float32, device=q.device)
    with torch.cuda.device(q.device):
        _lib.check(_lib.load().sqx_awq_dequantize(qc.data_ptr(), gsc.data_ptr(), sc.data_ptr(), rows, cols,
                                                  quant.group_size, out.data_ptr(), _stream(qc)), "awq_dequantize")
    return out


_tiled_cache = _device.TensorKeyedCache()


def awq_linear(x: Tensor, quant: AWQQuant, bias: Tensor | None = None) -> Tensor:
    """W4A16 linear with an AWQ weight, ``y = x @ W_eff^T (+ bias)`` in ``x.dtype`` (awq.py:184-192),
    computed as the int4 linear of ``x / s`` against the codes of ``W * s``."""
    _lib.require_device(x, quant.q, quant.chan_scale, bias, fn="awq_linear")
    g = quant.group_size
    try:
        tiled_group(g)
    except ValueError:
        raise ValueError(f"awq_linear: group_size={g} is not supported by the MI355X kernels (one of "
                         f"{TILED_GROUPS} or a multiple of 32)") from None
    tw = _tiled_cache.get((quant.q, quant.group_scales), (g,), lambda: tile_int4(quant.q, quant.group_scales, None, g))
    return awq_linear_tiled(x, tw, quant.chan_scale, bias)


def awq_linear_tiled(x: Tensor, tw: Int4Tiled, chan_scale: Tensor, bias: Tensor | None = None) -> Tensor:
    """:func:`awq_linear` on a tiled weight (the codes and group scales of ``W * s`` re-laid by
    ``tile_int4``) and its per-input-channel scale ``s``."""
    _lib.require_device(x, tw.wt, chan_scale, bias, fn="awq_linear")
    if x.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise TypeError(f"awq_linear takes fp32, bf16 or fp16 activations, got {x.dtype}")
    g = tw.group_size
    s = chan_scale.to(torch.float32).contiguous()
    if x.dtype == torch.float32:
        return int4_linear_tiled_f32(x, tw, bias, col_scale=s)
    *batch, k = x.shape
    x2 = x.reshape(-1, k)
    if not x2.is_contiguous() or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    m = x2.shape[0]
    lib = _lib.load()
    with torch.cuda.device(x.device):
        if m <= 16 and m * (-(-k // 128) * 128 + 8) * 2 <= 66 * 1024:  # the GEMV's LDS copy of the rows
            y = torch.empty(m, tw.rows, dtype=x.dtype, device=x.device)
            b = None if bias is None else bias.to(x.dtype).contiguous()
            _lib.check(lib.sqx_int4_linear_colscaled(tw.wt.data_ptr(), tw.st.data_ptr(), None, _lib.DTYPE_F32,
                                                     x2.data_ptr(), _lib.sqx_dtype(x.dtype), s.data_ptr(), y.data_ptr(),
                                                     _lib.ptr(b), m, tw.rows, tw.cols, g, 0, _stream(x2)), "awq_linear")
            return y.reshape(*batch, tw.rows)
        xs = torch.empty_like(x2)
        _lib.check(lib.sqx_scale_columns(x2.data_ptr(), _lib.sqx_dtype(x.dtype), s.data_ptr(), m, k, xs.data_ptr(),
                                         _stream(x2)), "awq_linear")
    return int4_linear_tiled(xs, tw, bias).reshape(*batch, tw.rows)

