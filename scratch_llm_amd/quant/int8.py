"""INT8 on MI355X — the API of ``scratch_llm.quant.int8``.

Same names, signatures, defaults and return types as ``src/scratch_llm/quant/int8.py`` (cited per
function), computed by the HIP kernels of ``libsqx_hip.so`` on ROCm device tensors. Like the
reference, the quantizers compute in the input's dtype, and the kernels round each intermediate to
that dtype where torch does, so codes, scales and zero-points are bit-identical for float32,
bfloat16 and float16 inputs. ``w8a8_linear`` accumulates exactly in int32 on int8 MFMA and applies
the reference's fp32 epilogue, so its output is bit-identical too.

Beyond the reference API, :func:`int8_weight_linear` is BASELINE config 1's weight-only linear
``x @ (q * s).to(x.dtype).T`` on a tiled copy of the codes.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor

from scratch_llm_amd import _lib
from scratch_llm_amd.quant import _device

__all__ = [
    "Int8Tiled",
    "dequantize_affine",
    "dequantize_symmetric",
    "fake_quant_affine",
    "fake_quant_symmetric",
    "int8_weight_linear",
    "int8_linear_tiled",
    "mse",
    "quantize_affine",
    "quantize_symmetric",
    "sqnr_db",
    "tile_int8",
    "w8a8_linear",
]

_SYM_QMAX = 127
_AFF_QMIN = 0
_AFF_QMAX = 255
_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def sqnr_db(x: Tensor, x_hat: Tensor) -> float:
    """``10*log10(P_signal / P_noise)`` in float64; ``+inf`` for an exact reconstruction (int8.py:82-91)."""
    sig = (x.double() ** 2).sum()
    noise = ((x.double() - x_hat.double()) ** 2).sum()
    if noise.item() == 0.0:
        return float("inf")
    return (10.0 * torch.log10(sig / noise)).item()


def mse(x: Tensor, x_hat: Tensor) -> float:
    """Mean squared reconstruction error in float64 (int8.py:94-96)."""
    return ((x.double() - x_hat.double()) ** 2).mean().item()


def _view(shape: torch.Size, axis: int | None) -> tuple[int, int, int, list[int]]:
    """[A, B, C] view with B the kept axis, and the keepdim shape of the per-slice statistics.

    As in the reference (int8.py:120-121), the kept dim is the one whose index equals ``axis``: a
    negative or out-of-range ``axis`` keeps none, i.e. one scale over the whole tensor with a
    keepdim shape of ones; ``axis=None`` gives a 0-dim scale."""
    n = 1
    for d in shape:
        n *= int(d)
    if axis is None:
        return 1, 1, max(n, 1), []
    nd = len(shape)
    if not 0 <= axis < nd:
        return 1, 1, max(n, 1), [1] * nd
    a = 1
    for d in shape[:axis]:
        a *= int(d)
    c = 1
    for d in shape[axis + 1:]:
        c *= int(d)
    keep = [1] * nd
    keep[axis] = int(shape[axis])
    return a, int(shape[axis]), c, keep


def _input(x: Tensor, fn: str) -> Tensor:
    _lib.require_device(x, fn=fn)
    if x.dtype not in _DTYPES:
        raise TypeError(f"{fn}: the MI355X kernels take float32, bfloat16 or float16 inputs, got {x.dtype}")
    return x.detach().contiguous()


def _workspace(dev: torch.device) -> Tensor:
    return torch.empty(_lib.load().sqx_int8_workspace_bytes() // 4, dtype=torch.float32, device=dev)


# --------------------------------------------------------------------------------------------
# Symmetric (int8.py:102-136)
# --------------------------------------------------------------------------------------------
def quantize_symmetric(x: Tensor, axis: int | None = None, eps: float = 1e-12) -> tuple[Tensor, Tensor]:
    """Symmetric INT8 (int8.py:102-125): ``s = (amax / 127).clamp_min(eps)``,
    ``q = round(x / s).clamp(-127, 127)``; ``axis`` is the kept dim (amax over all others, keepdim),
    ``None`` for one per-tensor scale. Returns ``(q int8, s)`` with ``s`` in ``x``'s dtype."""
    xc = _input(x, "quantize_symmetric")
    a, b, c, keep = _view(xc.shape, axis)
    q = torch.empty(xc.shape, dtype=torch.int8, device=xc.device)
    s = torch.empty(keep, dtype=xc.dtype, device=xc.device)
    if xc.numel() == 0:
        raise RuntimeError("quantize_symmetric: empty tensor (max of an empty tensor is undefined)")
    ws = _workspace(xc.device) if b == 1 else None
    with torch.cuda.device(xc.device):
        _lib.check(_lib.load().sqx_int8_quantize_sym(
            xc.data_ptr(), _lib.sqx_dtype(xc.dtype), a, b, c, eps, q.data_ptr(), s.data_ptr(), _lib.ptr(ws),
            0 if ws is None else ws.numel() * 4, _lib.stream_ptr(xc.device)), "quantize_symmetric")
    return q, s


def _broadcast_view(q: Tensor, s: Tensor) -> tuple[int, int, int, Tensor, torch.Size]:
    """[A, B, C] view of q in which s (broadcastable) has one value per B index; falls back to an
    elementwise scale when s is not a per-tensor or single-axis keepdim tensor."""
    out_shape = torch.broadcast_shapes(q.shape, s.shape)
    if s.numel() == 1:
        return 1, 1, max(q.numel(), 1), s.reshape(()).contiguous(), out_shape
    if q.shape == out_shape and s.dim() == q.dim():
        axes = [i for i, d in enumerate(s.shape) if d != 1]
        if len(axes) == 1 and s.shape[axes[0]] == q.shape[axes[0]]:
            a, b, c, _ = _view(q.shape, axes[0])
            return a, b, c, s.contiguous(), out_shape
    n = 1
    for d in out_shape:
        n *= int(d)
    return 1, max(n, 1), 1, s.expand(out_shape).contiguous(), out_shape


def dequantize_symmetric(q: Tensor, s: Tensor) -> Tensor:
    """``x_hat = q.to(s.dtype) * s`` (int8.py:128-130)."""
    _lib.require_device(q, s, fn="dequantize_symmetric")
    if s.dtype not in _DTYPES:
        raise TypeError(f"dequantize_symmetric: scale dtype {s.dtype} not supported")
    qx = q.to(torch.int8)
    if torch.broadcast_shapes(q.shape, s.shape) != q.shape:
        qx = qx.expand(torch.broadcast_shapes(q.shape, s.shape))
    qx = qx.contiguous()
    a, b, c, sv, shape = _broadcast_view(qx, s)
    out = torch.empty(shape, dtype=s.dtype, device=qx.device)
    if out.numel():
        with torch.cuda.device(qx.device):
            _lib.check(_lib.load().sqx_int8_dequantize_sym(qx.data_ptr(), a, b, c, sv.data_ptr(), _lib.sqx_dtype(s.dtype),
                                                           out.data_ptr(), _lib.stream_ptr(qx.device)),
                       "dequantize_symmetric")
    return out


def fake_quant_symmetric(x: Tensor, axis: int | None = None) -> Tensor:
    """Round trip ``x -> quantize -> dequantize`` under the symmetric scheme (int8.py:133-136)."""
    q, s = quantize_symmetric(x, axis=axis)
    return dequantize_symmetric(q, s)


# --------------------------------------------------------------------------------------------
# Asymmetric affine (int8.py:142-183)
# --------------------------------------------------------------------------------------------
def quantize_affine(x: Tensor, axis: int | None = None, eps: float = 1e-12) -> tuple[Tensor, Tensor, Tensor]:
    """Asymmetric affine INT8 onto ``[0, 255]`` (int8.py:142-172). Returns ``(q uint8, s, z)`` with the
    float scale and integer-valued zero-point in ``x``'s dtype, keepdim-shaped per ``axis``."""
    xc = _input(x, "quantize_affine")
    a, b, c, keep = _view(xc.shape, axis)
    if xc.numel() == 0:
        raise RuntimeError("quantize_affine: empty tensor (min of an empty tensor is undefined)")
    q = torch.empty(xc.shape, dtype=torch.uint8, device=xc.device)
    s = torch.empty(keep, dtype=xc.dtype, device=xc.device)
    z = torch.empty(keep, dtype=xc.dtype, device=xc.device)
    ws = _workspace(xc.device) if b == 1 else None
    with torch.cuda.device(xc.device):
        _lib.check(_lib.load().sqx_int8_quantize_affine(
            xc.data_ptr(), _lib.sqx_dtype(xc.dtype), a, b, c, eps, q.data_ptr(), s.data_ptr(), z.data_ptr(),
            _lib.ptr(ws), 0 if ws is None else ws.numel() * 4, _lib.stream_ptr(xc.device)), "quantize_affine")
    return q, s, z


def dequantize_affine(q: Tensor, s: Tensor, z: Tensor) -> Tensor:
    """``x_hat = (q.to(s.dtype) - z) * s`` (int8.py:175-177)."""
    _lib.require_device(q, s, z, fn="dequantize_affine")
    if s.dtype not in _DTYPES:
        raise TypeError(f"dequantize_affine: scale dtype {s.dtype} not supported")
    shape = torch.broadcast_shapes(q.shape, s.shape, z.shape)
    qx = q.to(torch.uint8).expand(shape).contiguous()
    sz = torch.broadcast_shapes(s.shape, z.shape)
    s2 = s.expand(sz)
    z2 = z.to(s.dtype).expand(sz)
    a, b, c, sv, _ = _broadcast_view(qx, s2)
    _, _, _, zv, _ = _broadcast_view(qx, z2)
    out = torch.empty(shape, dtype=s.dtype, device=qx.device)
    if out.numel():
        with torch.cuda.device(qx.device):
            _lib.check(_lib.load().sqx_int8_dequantize_affine(qx.data_ptr(), a, b, c, sv.data_ptr(), zv.data_ptr(),
                                                              _lib.sqx_dtype(s.dtype), out.data_ptr(),
                                                              _lib.stream_ptr(qx.device)), "dequantize_affine")
    return out


def fake_quant_affine(x: Tensor, axis: int | None = None) -> Tensor:
    """Round trip under the asymmetric affine scheme (int8.py:180-183)."""
    q, s, z = quantize_affine(x, axis=axis)
    return dequantize_affine(q, s, z)


# --------------------------------------------------------------------------------------------
# W8A8 linear (int8.py:189-213)
# --------------------------------------------------------------------------------------------
def w8a8_linear(x: Tensor, w: Tensor) -> Tensor:
    """Fake-quant W8A8 linear ``Y ~ X @ W.T`` (int8.py:189-213): per-token symmetric int8 ``x``,
    per-output-channel symmetric int8 ``w``, exact int32 accumulation, then
    ``acc.to(fp32) * (s_x * s_w)``. ``x`` is ``[..., in]``, ``w`` is ``[out, in]``."""
    *batch, in_features = x.shape
    x2d = x.reshape(-1, in_features)
    q_x, s_x = quantize_symmetric(x2d, axis=0)
    q_w, s_w = quantize_symmetric(w, axis=0)
    m, n, k = q_x.shape[0], q_w.shape[0], in_features
    out_dtype = torch.promote_types(torch.float32, torch.promote_types(s_x.dtype, s_w.dtype))
    y = torch.empty(m, n, dtype=torch.float32, device=q_x.device)
    with torch.cuda.device(q_x.device):
        _lib.check(_lib.load().sqx_w8a8_gemm(q_x.data_ptr(), s_x.data_ptr(), _lib.sqx_dtype(s_x.dtype), q_w.data_ptr(),
                                             s_w.data_ptr(), _lib.sqx_dtype(s_w.dtype), y.data_ptr(), m, n, k,
                                             _lib.stream_ptr(q_x.device)), "w8a8_linear")
    return y.to(out_dtype).reshape(*batch, w.shape[0])


# --------------------------------------------------------------------------------------------
# Weight-only int8 linear
# --------------------------------------------------------------------------------------------
@dataclass(frozen=True)
class Int8Tiled:
    """Symmetric int8 codes re-laid for the linear kernels (1 KiB per 16-row x 64-column block)
    with the per-row fp32 scale."""

    wt: Tensor
    scale: Tensor
    rows: int
    cols: int


def tile_int8(q: Tensor, s: Tensor) -> Int8Tiled:
    """Re-lay ``q [out, in]`` (int8 codes) with per-row scales ``s`` (``[out]`` or ``[out, 1]``)."""
    if q.dim() != 2:
        raise ValueError(f"expected 2-D codes, got shape {tuple(q.shape)}")
    rows, cols = q.shape
    _lib.require_device(q, s, fn="tile_int8")
    if s.numel() not in (1, rows):
        raise ValueError(f"scale has {s.numel()} elements; expected 1 or {rows} (one per output row)")
    sc = s.to(torch.float32).reshape(-1).expand(rows).contiguous()
    lib = _lib.load()
    wt = torch.empty(lib.sqx_int8_tiled_weight_bytes(rows, cols), dtype=torch.uint8, device=q.device)
    qc = q.to(torch.int8).contiguous()
    with torch.cuda.device(q.device):
        _lib.check(lib.sqx_int8_tile(qc.data_ptr(), rows, cols, wt.data_ptr(), _lib.stream_ptr(q.device)), "tile_int8")
    return Int8Tiled(wt, sc, rows, cols)


def untile_int8(tw: Int8Tiled) -> Tensor:
    """The int8 codes ``[out, in]`` back from a tiled weight (``sqx_int8_untile``, the exact inverse of
    :func:`tile_int8`)."""
    dev = _lib.require_device(tw.wt, fn="untile_int8")
    q = torch.empty(tw.rows, tw.cols, dtype=torch.int8, device=dev)
    with torch.cuda.device(dev):
        _lib.check(_lib.load().sqx_int8_untile(tw.wt.data_ptr(), tw.rows, tw.cols, q.data_ptr(), _lib.stream_ptr(dev)),
                   "untile_int8")
    return q


def int8_linear_tiled(x: Tensor, tw: Int8Tiled, bias: Tensor | None = None, k_slices: int | None = None) -> Tensor:
    """``x @ (q * s).T (+ bias)`` for a tiled int8 weight; ``x`` bf16 / fp16 ``[..., in]``."""
    *batch, k = x.shape
    if k != tw.cols:
        raise ValueError(f"x has in_features={k}, weight expects {tw.cols}")
    dev = _lib.require_device(x, tw.wt, bias, fn="int8_linear")
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"int8_linear takes bf16 or fp16 activations, got {x.dtype}")
    x2 = x.reshape(-1, k)
    if not x2.is_contiguous() or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    m = x2.shape[0]
    y = torch.empty(m, tw.rows, dtype=x.dtype, device=dev)
    b = None if bias is None else bias.to(x.dtype).contiguous()
    with torch.cuda.device(dev):
        _lib.check(_lib.load().sqx_int8_linear(tw.wt.data_ptr(), tw.scale.data_ptr(), x2.data_ptr(),
                                               _lib.sqx_dtype(x.dtype), y.data_ptr(), _lib.ptr(b), m, tw.rows, tw.cols,
                                               0 if k_slices is None else int(k_slices), _lib.stream_ptr(dev)),
                   "int8_linear")
    return y.reshape(*batch, tw.rows)


_tiled_cache = _device.TensorKeyedCache()


def int8_weight_linear(x: Tensor, q: Tensor, s: Tensor, bias: Tensor | None = None) -> Tensor:
    """``F.linear(x, dequantize_symmetric(q, s).to(x.dtype), bias)`` for per-row
    symmetric int8 codes ``q [out, in]`` and scales ``s [out, 1]`` (``quantize_symmetric(W, axis=0)``),
    without materialising the weight. bf16 / fp16 ``x``; output in ``x.dtype``."""
    tw = _tiled_cache.get((q, s), (), lambda: tile_int8(q, s))
    return int8_linear_tiled(x, tw, bias)
