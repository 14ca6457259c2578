"""Per-output-channel FP8 (E4M3) weights and the W8A8 linear on MI355X — the API of
``scratch_llm.quant.fp8_weights``.

Same names, constants, signatures, return types and ``ValueError`` messages as
``src/scratch_llm/quant/fp8_weights.py`` (cited per function), computed by the HIP kernels in
``libsqx_hip.so`` on ROCm device tensors. Codes are ``torch.float8_e4m3fn`` (OCP E4M3, the format
gfx950's FP8 conversions and MFMA read), bit-identical to the reference's casts.

Differences from the reference, all on purpose:
* CPU tensors raise ``RuntimeError`` (the reference's ``Fp8Linear`` falls back to its float64 oracle
  on the CPU; this package has no host path). ``fp8_linear_reference`` lives in the test oracle.
* ``fp8_linear`` does not call ``torch._scaled_mm``: the library's linear decodes both E4M3 operands
  exactly to bf16 and accumulates the exact products in fp32 (``sqx_fp8_linear``), which keeps the
  result inside the reference's own derived error bound; hipBLASLt's FP8 GEMM on this GPU does not
  (its MFMA aligns the products of a step with a limited-width adder). ``use_fast_accum`` is accepted
  and changes nothing: the accumulator is fp32 either way.
"""

from __future__ import annotations

import torch
from torch import Tensor, nn

from scratch_llm_amd import _lib
from scratch_llm_amd.quant import _device

__all__ = [
    "DEFAULT_FAST_ACCUM",
    "DEFAULT_SKIP",
    "E4M3_MAX",
    "E4M3_MIN_NORMAL",
    "E4M3_MIN_SUBNORMAL",
    "E4M3_NAN_ABOVE",
    "E4M3_UNIT_ROUNDOFF",
    "FP8_DTYPE",
    "MIN_SCALE",
    "Fp8Linear",
    "Fp8Tiled",
    "convert_linears_to_fp8",
    "dequantize",
    "fp8_linear",
    "fp8_linear_tiled",
    "quantize_per_channel",
    "quantize_per_token",
    "rowwise_scaled_mm_supported",
    "saturating_cast_e4m3",
    "tile_fp8",
]

FP8_DTYPE = torch.float8_e4m3fn
E4M3_MAX = 448.0
E4M3_NAN_ABOVE = 464.0
E4M3_UNIT_ROUNDOFF = 0.0625
E4M3_MIN_NORMAL = 0.015625
E4M3_MIN_SUBNORMAL = 0.001953125
DEFAULT_FAST_ACCUM = False
MIN_SCALE = 1.0 / (E4M3_MAX * 512.0)
DEFAULT_SKIP = ("lm_head", "embed", "wte", "output")


def _float_input(t: Tensor) -> Tensor:
    if t.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        t = t.to(torch.float32)
    return t.contiguous()


def saturating_cast_e4m3(v: Tensor) -> Tensor:
    """``v.clamp(-448, 448).to(float8_e4m3fn)`` (fp8_weights.py:117-124): round to nearest even,
    saturating instead of producing NaN above 464. Any shape."""
    dev = _lib.require_device(v, fn="saturating_cast_e4m3")
    x = _float_input(v)
    codes = torch.empty(x.shape, dtype=torch.uint8, device=dev)
    one = torch.ones(1, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.load().sqx_fp8_quantize_heads(
            _lib.ptr(x), _lib.sqx_dtype(x.dtype), 1, 1, x.numel(), _lib.ptr(one), _lib.ptr(codes), None,
            _lib.stream_ptr(dev),
        )
    _lib.check(rc, "saturating_cast_e4m3")
    return codes.view(FP8_DTYPE)


def _quantize_rows(x: Tensor, fn: str) -> tuple[Tensor, Tensor]:
    dev = _lib.require_device(x, fn=fn)
    xx = _float_input(x)
    rows, cols = xx.shape
    codes = torch.empty(rows, cols, dtype=torch.uint8, device=dev)
    scale = torch.empty(rows, 1, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.load().sqx_fp8_quantize_rows(
            _lib.ptr(xx), _lib.sqx_dtype(xx.dtype), rows, cols, _lib.ptr(codes), _lib.ptr(scale), _lib.stream_ptr(dev)
        )
    _lib.check(rc, fn)
    return codes.view(FP8_DTYPE), scale


def quantize_per_channel(w: Tensor) -> tuple[Tensor, Tensor]:
    """Weight ``(N, K)`` -> E4M3 codes ``(N, K)`` and fp32 scale ``(N, 1)``, ``amax_k / 448`` floored at
    ``MIN_SCALE`` (fp8_weights.py:133-143)."""
    if w.ndim != 2:
        raise ValueError(f"weight must be 2-D (N, K), got shape {tuple(w.shape)}")
    return _quantize_rows(w, "quantize_per_channel")


def quantize_per_token(x: Tensor) -> tuple[Tensor, Tensor]:
    """Activation ``(M, K)`` -> E4M3 codes and fp32 scale ``(M, 1)`` (fp8_weights.py:146-155)."""
    if x.ndim != 2:
        raise ValueError(f"activation must be 2-D (M, K), got shape {tuple(x.shape)}")
    return _quantize_rows(x, "quantize_per_token")


def dequantize(codes: Tensor, scale: Tensor) -> Tensor:
    """``codes * scale`` in fp32 (fp8_weights.py:158-160) for codes ``(N, K)`` with a per-row scale
    ``(N, 1)`` (the pairs the quantizers return)."""
    if codes.ndim != 2 or scale.numel() != codes.shape[0]:
        raise ValueError(f"expected codes (N, K) and a scale of N elements, got {tuple(codes.shape)} and {tuple(scale.shape)}")
    dev = _lib.require_device(codes, scale, fn="dequantize")
    c = codes.contiguous().view(torch.uint8)
    s = scale.to(torch.float32).contiguous()
    out = torch.empty(codes.shape, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.load().sqx_fp8_dequantize_rows(_lib.ptr(c), _lib.ptr(s), codes.shape[0], codes.shape[1], _lib.ptr(out),
                                                 _lib.stream_ptr(dev))
    _lib.check(rc, "dequantize")
    return out


def rowwise_scaled_mm_supported(device_index: int = 0) -> bool:
    """Whether per-token x per-channel scales run fused on this device (fp8_weights.py:163-186): they
    always do in ``sqx_fp8_linear``, on any visible ROCm device."""
    return torch.cuda.is_available() and device_index < torch.cuda.device_count()


class Fp8Tiled:
    """E4M3 codes re-laid for ``sqx_fp8_linear`` (1 KiB blocks of 16 rows x 64 columns) with the fp32
    per-row scales."""

    def __init__(self, wt: Tensor, scale: Tensor, rows: int, cols: int) -> None:
        self.wt, self.scale, self.rows, self.cols = wt, scale, rows, cols

    @property
    def nbytes(self) -> int:
        return self.wt.numel() + self.scale.numel() * 4


def tile_fp8(weight_codes: Tensor, weight_scale: Tensor) -> Fp8Tiled:
    """Re-lay ``(N, K)`` E4M3 codes and their ``(N, 1)`` scale for the linear kernel."""
    if weight_codes.ndim != 2:
        raise ValueError(f"weight must be 2-D (N, K), got shape {tuple(weight_codes.shape)}")
    dev = _lib.require_device(weight_codes, weight_scale, fn="tile_fp8")
    rows, cols = weight_codes.shape
    if weight_scale.numel() != rows:
        raise ValueError(f"weight_scale has {weight_scale.numel()} elements, expected {rows}")
    lib = _lib.load()
    wt = torch.empty(lib.sqx_fp8_tiled_weight_bytes(rows, cols), dtype=torch.uint8, device=dev)
    c = weight_codes.contiguous().view(torch.uint8)
    with torch.cuda.device(dev):
        rc = lib.sqx_fp8_tile(_lib.ptr(c), rows, cols, _lib.ptr(wt), _lib.stream_ptr(dev))
    _lib.check(rc, "tile_fp8")
    return Fp8Tiled(wt, weight_scale.to(torch.float32).reshape(rows).contiguous(), rows, cols)


_tiled_cache = _device.TensorKeyedCache()


def fp8_linear_tiled(x: Tensor, tw: Fp8Tiled, bias: Tensor | None = None, *, out_dtype: torch.dtype = torch.bfloat16,
                     k_slices: int | None = None) -> Tensor:
    """``fp8_linear`` on a tiled weight: x ``(..., K)`` quantized per token, E4M3 x E4M3 with exact
    products and fp32 accumulation, ``* s_x[m] * s_w[n] (+ bias)``, cast to ``out_dtype``."""
    *batch, k = x.shape
    if k != tw.cols:
        raise ValueError(f"activation last dim {k} != weight K {tw.cols}")
    dev = _lib.require_device(x, tw.wt, bias, fn="fp8_linear")
    if out_dtype not in (torch.bfloat16, torch.float32, torch.float16):
        raise TypeError(f"out_dtype {out_dtype} is not supported")
    x2 = _float_input(x.reshape(-1, k))
    m = x2.shape[0]
    lib = _lib.load()
    ydt = torch.bfloat16 if out_dtype == torch.bfloat16 else torch.float32
    y = torch.empty(m, tw.rows, dtype=ydt, device=dev)
    ws = torch.empty(max(-(-int(lib.sqx_fp8_linear_workspace_bytes(m, tw.rows, k)) // 4), 4), dtype=torch.float32,
                     device=dev)
    b = None
    if bias is not None and ydt == torch.bfloat16:
        b = bias.to(torch.bfloat16).contiguous()
    with torch.cuda.device(dev):
        rc = lib.sqx_fp8_linear(
            _lib.ptr(tw.wt), _lib.ptr(tw.scale), _lib.ptr(x2), _lib.sqx_dtype(x2.dtype), _lib.ptr(y), _lib.sqx_dtype(ydt),
            _lib.ptr(b), m, tw.rows, tw.cols, 0 if k_slices is None else int(k_slices), ws.data_ptr(), ws.numel() * 4,
            _lib.stream_ptr(dev),
        )
    _lib.check(rc, "fp8_linear")
    if bias is not None and ydt != torch.bfloat16:
        y = y + bias.to(torch.float32)
    return y.to(out_dtype).reshape(*batch, tw.rows)


def fp8_linear(
    x: Tensor,
    weight_codes: Tensor,
    weight_scale: Tensor,
    bias: Tensor | None = None,
    *,
    out_dtype: torch.dtype = torch.bfloat16,
    use_fast_accum: bool = DEFAULT_FAST_ACCUM,
) -> Tensor:
    """``x @ dequant(weight)^T + bias`` with per-token E4M3 activations (fp8_weights.py:211-262).
    ``use_fast_accum`` is accepted for the reference's signature; the accumulator is fp32 regardless."""
    if x.is_cpu:
        raise RuntimeError(
            "fp8_linear needs a ROCm device (the MI355X kernels have no CPU path); the reference's "
            "fp8_linear_reference is the CPU oracle"
        )
    n, k = weight_codes.shape
    if x.shape[-1] != k:
        raise ValueError(f"activation last dim {x.shape[-1]} != weight K {k}")
    if k % 16 != 0:
        raise ValueError(f"torch._scaled_mm requires K % 16 == 0, got K={k}")
    tw = _tiled_cache.get((weight_codes, weight_scale), (), lambda: tile_fp8(weight_codes, weight_scale))
    return fp8_linear_tiled(x, tw, bias, out_dtype=out_dtype)


class Fp8Linear(nn.Module):
    """Drop-in for ``nn.Linear`` holding E4M3 codes and a per-channel scale (fp8_weights.py:289-358),
    plus the tiled copy the kernel streams."""

    weight_codes: Tensor
    weight_scale: Tensor
    bias: Tensor | None

    def __init__(self, weight_codes: Tensor, weight_scale: Tensor, bias: Tensor | None = None, *,
                 out_dtype: torch.dtype = torch.bfloat16, use_fast_accum: bool = DEFAULT_FAST_ACCUM) -> None:
        super().__init__()
        self.register_buffer("weight_codes", weight_codes)
        self.register_buffer("weight_scale", weight_scale)
        self.register_buffer("bias", bias)
        self.out_dtype = out_dtype
        self.use_fast_accum = use_fast_accum
        self.out_features, self.in_features = weight_codes.shape
        self._tiled: Fp8Tiled | None = None

    @classmethod
    def from_linear(cls, linear: nn.Linear, *, out_dtype: torch.dtype | None = None,
                    use_fast_accum: bool = DEFAULT_FAST_ACCUM) -> "Fp8Linear":
        codes, scale = quantize_per_channel(linear.weight.data)
        bias = None if linear.bias is None else linear.bias.data.clone()
        return cls(codes, scale, bias, out_dtype=out_dtype or linear.weight.dtype, use_fast_accum=use_fast_accum)

    def dequantized_weight(self) -> Tensor:
        """``(N, K)`` fp32: what the GEMM sees."""
        return dequantize(self.weight_codes, self.weight_scale)

    def forward(self, x: Tensor) -> Tensor:
        _lib.require_device(x, self.weight_codes, fn="Fp8Linear")
        if self.in_features % 16 != 0:
            raise ValueError(f"torch._scaled_mm requires K % 16 == 0, got K={self.in_features}")
        if self._tiled is None or self._tiled.wt.device != self.weight_codes.device:
            self._tiled = tile_fp8(self.weight_codes, self.weight_scale)
        return fp8_linear_tiled(x, self._tiled, self.bias, out_dtype=self.out_dtype)


def convert_linears_to_fp8(root: nn.Module, *, skip: tuple[str, ...] = DEFAULT_SKIP, min_in_features: int = 16,
                           use_fast_accum: bool = DEFAULT_FAST_ACCUM) -> list[str]:
    """Replace every ``nn.Linear`` under ``root`` with :class:`Fp8Linear`, in place; returns the
    qualified names replaced (fp8_weights.py:368-400: a child whose local name contains a ``skip``
    entry, or whose ``in_features`` is not a multiple of ``min_in_features``, is left alone). The walk
    is the one every converter of this package shares (``modules._convert``), restricted to
    ``nn.Linear`` as the reference's FP8 converter is."""
    from scratch_llm_amd.quant import modules  # the module converters import this one's neighbours

    return modules._convert(
        root, lambda m: Fp8Linear.from_linear(m, use_fast_accum=use_fast_accum),
        lambda m: isinstance(m, nn.Linear) and m.in_features % min_in_features == 0, skip)
