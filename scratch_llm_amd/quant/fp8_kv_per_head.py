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
    """The decode-contract KV cache of fp8_kv_per_head.py:120-223 (``length`` / ``append`` / ``get`` /
    ``advance``, ``scales`` / ``set_scales``, ``codes``, saturation counters, ``kv_bytes``) on a
    device-resident layout of its own.

    * **Storage.** Each layer owns one uint8 buffer ``[2, B, H, capacity, D]`` (plane 0 holds K codes,
      plane 1 V codes), allocated by the first append and grown by doubling ``capacity`` along the
      token axis when an append would not fit, so n appends copy O(n) tokens in total. The layer's
      filled token count is ``_fill[layer]``; ``(B, H, D)`` are fixed by its first append.
    * **Scales.** One fp32 device tensor ``[n_layers, 2, H]``; a layer's pair is either installed
      (``set_scales``) or calibrated from the first block appended to it (``per_head_scale``) and is
      static afterwards, as the reference's calibrate-once contract states.
    * **Saturation.** The quantize kernel adds the count of clamped elements straight into a device
      int64 pair ``[K, V]``, so an append issues device work only; reading ``k_saturated`` /
      ``v_saturated`` / ``saturated_fraction()`` synchronises.
    * ``kv_bytes`` counts the stored code bytes plus 4 bytes per head for each scale vector a layer
      holds; ``get`` returns freshly dequantized ``(K, V)`` in ``dtype`` and ``codes`` fresh
      ``float8_e4m3fn`` copies of the filled region.
    """

    def __init__(self, n_layers: int, *, dtype: torch.dtype = torch.float32) -> None:
        if n_layers <= 0:
            raise ValueError("n_layers must be positive")
        self.n_layers = n_layers
        self.dtype = dtype
        self._buf: list[Tensor | None] = [None] * n_layers
        self._fill = [0] * n_layers
        self._scale_t: Tensor | None = None  # [n_layers, 2, H] fp32, created with the first scales
        self._has_scale = [False] * n_layers
        self._sat: Tensor | None = None  # int64 [2] on the cache's device
        self._tokens = 0

    # ------------------------------------------------------------------ bookkeeping
    @property
    def length(self) -> int:
        return self._tokens

    def advance(self, n: int) -> None:
        self._tokens += n

    @property
    def n_elements(self) -> int:
        """Code bytes stored across layers (one byte per K or V element)."""
        return sum(0 if b is None else 2 * b.shape[1] * b.shape[2] * f * b.shape[4] for b, f in zip(self._buf, self._fill))

    @property
    def kv_bytes(self) -> int:
        heads = 0 if self._scale_t is None else self._scale_t.shape[2]
        return self.n_elements + sum(self._has_scale) * 2 * heads * 4

    def _sat_counts(self) -> tuple[int, int]:
        if self._sat is None:
            return 0, 0
        k, v = self._sat.tolist()
        return int(k), int(v)

    @property
    def k_saturated(self) -> int:
        return self._sat_counts()[0]

    @property
    def v_saturated(self) -> int:
        return self._sat_counts()[1]

    def saturated_fraction(self) -> float:
        n = self.n_elements
        return 0.0 if n == 0 else sum(self._sat_counts()) / n

    # ------------------------------------------------------------------ scales
    def _scale_rows(self, heads: int, device: torch.device) -> Tensor:
        if self._scale_t is None:
            self._scale_t = torch.zeros(self.n_layers, 2, heads, dtype=torch.float32, device=device)
        elif self._scale_t.shape[2] != heads:
            raise ValueError(f"this cache holds {self._scale_t.shape[2]} heads per layer, got {heads}")
        return self._scale_t

    def scales(self, layer: int) -> tuple[Tensor | None, Tensor | None]:
        if not self._has_scale[layer]:
            return None, None
        # copies: a later set_scales rewrites the device rows in place, and the reference hands out
        # tensors that a later install replaces rather than changes
        row = self._scale_t[layer].clone()
        return row[0].view(1, -1, 1, 1), row[1].view(1, -1, 1, 1)

    def set_scales(self, layer: int, k_scale: Tensor, v_scale: Tensor) -> None:
        for sc in (k_scale, v_scale):
            if sc.ndim != 4 or sc.shape[0] != 1 or sc.shape[2] != 1 or sc.shape[3] != 1:
                raise ValueError(f"scale must be (1, H, 1, 1), got {tuple(sc.shape)}")
        dev = _lib.require_device(k_scale, v_scale, fn="PerHeadFp8KVCache.set_scales")
        rows = self._scale_rows(k_scale.shape[1], dev)
        rows[layer, 0].copy_(k_scale.reshape(-1))
        rows[layer, 1].copy_(v_scale.reshape(-1))
        self._has_scale[layer] = True

    # ------------------------------------------------------------------ storage
    def _reserve(self, layer: int, like: Tensor, extra: int) -> Tensor:
        b, h, _, d = like.shape
        buf, fill = self._buf[layer], self._fill[layer]
        if buf is not None and tuple(buf.shape[1:3]) + (buf.shape[4],) != (b, h, d):
            raise ValueError(f"layer {layer} holds blocks of (B, H, D) = {(buf.shape[1], buf.shape[2], buf.shape[4])}, "
                             f"got {(b, h, d)}")
        cap = 0 if buf is None else buf.shape[3]
        if fill + extra > cap:
            new_cap = max(fill + extra, 2 * cap, 16)
            grown = torch.empty(2, b, h, new_cap, d, dtype=torch.uint8, device=like.device)
            if buf is not None and fill:
                grown[:, :, :, :fill].copy_(buf[:, :, :, :fill])
            self._buf[layer] = buf = grown
        return buf

    def append(self, layer: int, k_new: Tensor, v_new: Tensor) -> None:
        for blk in (k_new, v_new):
            if blk.ndim != 4:
                raise ValueError(f"KV block must be (B, H, T, D), got shape {tuple(blk.shape)}")
        if k_new.shape != v_new.shape:
            raise ValueError(f"K and V blocks differ in shape: {tuple(k_new.shape)} vs {tuple(v_new.shape)}")
        dev = _lib.require_device(k_new, v_new, fn="PerHeadFp8KVCache.append")
        if not self._has_scale[layer]:  # calibrate once, on this block
            self.set_scales(layer, per_head_scale(k_new), per_head_scale(v_new))
        if self._sat is None:
            self._sat = torch.zeros(2, dtype=torch.int64, device=dev)
        t = k_new.shape[2]
        buf = self._reserve(layer, k_new, t)
        f0 = self._fill[layer]
        kv_scales = self.scales(layer)
        for plane, (blk, sc) in enumerate(zip((k_new, v_new), kv_scales)):
            codes, _ = _quantize_into(blk, sc, self._sat[plane:plane + 1])
            buf[plane, :, :, f0:f0 + t].copy_(codes)
        self._fill[layer] = f0 + t

    def _planes(self, layer: int) -> tuple[Tensor, Tensor] | None:
        """Views of the filled K and V code planes (aliases of the internal buffer)."""
        buf, fill = self._buf[layer], self._fill[layer]
        if buf is None or fill == 0:
            return None
        return buf[0, :, :, :fill], buf[1, :, :, :fill]

    def get(self, layer: int) -> tuple[Tensor, Tensor] | None:
        planes = self._planes(layer)
        if planes is None:
            return None
        k_s, v_s = self.scales(layer)
        return dequantize_per_head(planes[0], k_s, self.dtype), dequantize_per_head(planes[1], v_s, self.dtype)

    def codes(self, layer: int) -> tuple[Tensor, Tensor] | None:
        """Fresh contiguous copies of the stored codes (``float8_e4m3fn``), as the reference's
        ``torch.cat`` returns: writing to them leaves the cache unchanged."""
        planes = self._planes(layer)
        if planes is None:
            return None
        return tuple(p.clone(memory_format=torch.contiguous_format).view(FP8_DTYPE) for p in planes)


def _quantize_into(x: Tensor, scale: Tensor, sat: Tensor) -> tuple[Tensor, Tensor]:
    """E4M3 codes (uint8) of a block at a per-head scale, with the clamped count added to ``sat``."""
    _check_scale(x, scale)
    dev = _lib.require_device(x, scale, sat, fn="quantize_per_head")
    xx = _f(x)
    b, h, t, d = xx.shape
    codes = torch.empty(xx.shape, dtype=torch.uint8, device=dev)
    s = scale.to(torch.float32).contiguous()
    with torch.cuda.device(dev):
        rc = _lib.load().sqx_fp8_quantize_heads(_lib.ptr(xx), _lib.sqx_dtype(xx.dtype), b, h, t * d, _lib.ptr(s),
                                                _lib.ptr(codes), _lib.ptr(sat), _lib.stream_ptr(dev))
    _lib.check(rc, "quantize_per_head")
    return codes, sat


def bf16_reference_bytes(n_elements: int) -> int:
    """Two bytes per element, no scales (:226-229)."""
    return n_elements * 2
