"""E4M3 KV cache with per-head scales on MI355X — the API of ``scratch_llm.quant.fp8_kv_per_head``.

Same names, signatures, return types and ``ValueError`` messages as
``src/scratch_llm/quant/fp8_kv_per_head.py`` (cited per function), computed by the HIP kernels of
``libsqx_hip.so`` on ROCm device tensors (CPU tensors raise ``RuntimeError``). Scales are
``amax / 448`` per head, reduced over batch, tokens and head_dim, floored at ``MIN_SCALE``; codes are
the saturating E4M3 cast of ``fp32(x) / scale``, bit-identical to the reference.

The decode step reads such a cache directly (``Int4DecodeLM.new_state(kv_dtype="fp8")``):
the attention kernel takes the codes and the per-head scales and never materialises fp32 K/V.
"""

from __future__ import annotations

import torch
from torch import Tensor

from scratch_llm_amd import _lib
from scratch_llm_amd.quant.fp8_weights import E4M3_MAX, FP8_DTYPE, MIN_SCALE  # noqa: F401  (re-exported names)

__all__ = [
    "PerHeadFp8KVCache",
    "bf16_reference_bytes",
    "dequantize_per_head",
    "per_head_amax",
    "per_head_scale",
    "quantize_per_head",
    "saturated_count",
]


def _f(x: Tensor) -> Tensor:
    if x.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        x = x.to(torch.float32)
    return x.contiguous()


def _head_stats(x: Tensor, want_scale: bool) -> Tensor:
    if x.ndim != 4:
        raise ValueError(f"KV block must be (B, H, T, D), got shape {tuple(x.shape)}")
    dev = _lib.require_device(x, fn="per_head_scale" if want_scale else "per_head_amax")
    xx = _f(x)
    b, h, t, d = xx.shape
    out = torch.empty(1, h, 1, 1, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.load().sqx_fp8_head_scale(
            _lib.ptr(xx), _lib.sqx_dtype(xx.dtype), b, h, t * d, None if want_scale else _lib.ptr(out),
            _lib.ptr(out) if want_scale else None, _lib.stream_ptr(dev),
        )
    _lib.check(rc, "per_head_scale")
    return out


def per_head_amax(x: Tensor) -> Tensor:
    """``(B, H, T, D) -> (1, H, 1, 1)``: the max magnitude anywhere in each head (fp8_kv_per_head.py:77-85)."""
    return _head_stats(x, want_scale=False)


def per_head_scale(x: Tensor) -> Tensor:
    """``amax / 448`` per head, floored at ``MIN_SCALE`` (fp8_kv_per_head.py:88-90)."""
    return _head_stats(x, want_scale=True)


def _check_scale(x: Tensor, scale: Tensor) -> None:
    """fp8_kv_per_head.py:110-117."""
    if x.ndim != 4:
        raise ValueError(f"KV block must be (B, H, T, D), got shape {tuple(x.shape)}")
    if tuple(scale.shape) != (1, x.shape[1], 1, 1):
        raise ValueError(
            f"per-head scale must have shape (1, H, 1, 1) = {(1, x.shape[1], 1, 1)}, "
            f"got {tuple(scale.shape)} — a scale of any other shape is not per-head"
        )


def _quantize(x: Tensor, scale: Tensor, count: bool) -> tuple[Tensor, Tensor | None]:
    _check_scale(x, scale)
    dev = _lib.require_device(x, scale, fn="quantize_per_head")
    xx = _f(x)
    b, h, t, d = xx.shape
    s = scale.to(torch.float32).contiguous()
    codes = torch.empty(xx.shape, dtype=torch.uint8, device=dev)
    sat = torch.zeros(1, dtype=torch.int64, device=dev) if count else None
    with torch.cuda.device(dev):
        rc = _lib.load().sqx_fp8_quantize_heads(
            _lib.ptr(xx), _lib.sqx_dtype(xx.dtype), b, h, t * d, _lib.ptr(s), _lib.ptr(codes), _lib.ptr(sat),
            _lib.stream_ptr(dev),
        )
    _lib.check(rc, "quantize_per_head")
    return codes.view(FP8_DTYPE), sat


def quantize_per_head(x: Tensor, scale: Tensor) -> Tensor:
    """``(B, H, T, D)`` -> E4M3 codes at a ``(1, H, 1, 1)`` scale; saturating, never NaN (:93-96)."""
    return _quantize(x, scale, count=False)[0]


def dequantize_per_head(codes: Tensor, scale: Tensor, dtype: torch.dtype = torch.float32) -> Tensor:
    """Codes back to ``dtype``: ``fp32(code) * scale`` (:99-101)."""
    if codes.ndim != 4:
        raise ValueError(f"KV block must be (B, H, T, D), got shape {tuple(codes.shape)}")
    dev = _lib.require_device(codes, scale, fn="dequantize_per_head")
    b, h, t, d = codes.shape
    c = codes.contiguous().view(torch.uint8)
    s = scale.to(torch.float32).contiguous()
    out = torch.empty(codes.shape, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.load().sqx_fp8_dequantize_heads(_lib.ptr(c), _lib.ptr(s), b, h, t * d, _lib.ptr(out),
                                                  _lib.stream_ptr(dev))
    _lib.check(rc, "dequantize_per_head")
    return out if dtype == torch.float32 else out.to(dtype)


def saturated_count(x: Tensor, scale: Tensor) -> int:
    """Elements of ``x`` the clamp moves, ``|x| > 448 * scale`` (:104-107). Synchronises to return an int."""
    _check_scale(x, scale)
    _, sat = _quantize(x, scale, count=True)
    return int(sat.item())


class PerHeadFp8KVCache:
    """Per-layer KV cache of E4M3 codes with static per-head scales (fp8_kv_per_head.py:120-223):
    the plain decode contract ``length`` / ``append`` / ``get`` / ``advance``, scales calibrated on
    the first block appended to a layer (or installed with ``set_scales``), clamped elements counted."""

    def __init__(self, n_layers: int, *, dtype: torch.dtype = torch.float32) -> None:
        if n_layers <= 0:
            raise ValueError("n_layers must be positive")
        self.n_layers = n_layers
        self.dtype = dtype
        self._k: list[list[Tensor]] = [[] for _ in range(n_layers)]
        self._v: list[list[Tensor]] = [[] for _ in range(n_layers)]
        self._k_scale: list[Tensor | None] = [None] * n_layers
        self._v_scale: list[Tensor | None] = [None] * n_layers
        self._length = 0
        self.kv_bytes = 0
        self.k_saturated = 0
        self.v_saturated = 0
        self.n_elements = 0

    @property
    def length(self) -> int:
        return self._length

    def scales(self, layer: int) -> tuple[Tensor | None, Tensor | None]:
        return self._k_scale[layer], self._v_scale[layer]

    def set_scales(self, layer: int, k_scale: Tensor, v_scale: Tensor) -> None:
        for s in (k_scale, v_scale):
            if s.ndim != 4 or s.shape[0] != 1 or s.shape[2] != 1 or s.shape[3] != 1:
                raise ValueError(f"scale must be (1, H, 1, 1), got {tuple(s.shape)}")
        self._k_scale[layer] = k_scale.to(torch.float32)
        self._v_scale[layer] = v_scale.to(torch.float32)
        self.kv_bytes += (k_scale.numel() + v_scale.numel()) * 4

    def saturated_fraction(self) -> float:
        if self.n_elements == 0:
            return 0.0
        return (self.k_saturated + self.v_saturated) / self.n_elements

    def _scale_for(self, layer: int, x: Tensor, which: str) -> Tensor:
        store = self._k_scale if which == "k" else self._v_scale
        scale = store[layer]
        if scale is None:
            scale = per_head_scale(x)
            store[layer] = scale
            self.kv_bytes += scale.numel() * 4
        return scale

    def append(self, layer: int, k_new: Tensor, v_new: Tensor) -> None:
        k_scale = self._scale_for(layer, k_new, "k")
        v_scale = self._scale_for(layer, v_new, "v")
        k_codes, k_sat = _quantize(k_new, k_scale, count=True)
        v_codes, v_sat = _quantize(v_new, v_scale, count=True)
        self.k_saturated += int(k_sat.item())
        self.v_saturated += int(v_sat.item())
        self._k[layer].append(k_codes)
        self._v[layer].append(v_codes)
        self.kv_bytes += k_codes.numel() + v_codes.numel()
        self.n_elements += k_codes.numel() + v_codes.numel()

    def get(self, layer: int) -> tuple[Tensor, Tensor] | None:
        if not self._k[layer]:
            return None
        k_scale, v_scale = self._k_scale[layer], self._v_scale[layer]
        assert k_scale is not None and v_scale is not None
        k = torch.cat(self._k[layer], dim=2)
        v = torch.cat(self._v[layer], dim=2)
        return dequantize_per_head(k, k_scale, self.dtype), dequantize_per_head(v, v_scale, self.dtype)

    def codes(self, layer: int) -> tuple[Tensor, Tensor] | None:
        if not self._k[layer]:
            return None
        return torch.cat(self._k[layer], dim=2), torch.cat(self._v[layer], dim=2)

    def advance(self, n: int) -> None:
        self._length += n


def bf16_reference_bytes(n_elements: int) -> int:
    """Two bytes per element, no scales (:226-229)."""
    return n_elements * 2
