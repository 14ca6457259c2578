"""NVFP4 / MXFP4 on MI355X — the API of ``scratch_llm.quant.nvfp4_mxfp4``.

Same names, signatures, defaults, payload classes (``NVFP4Tensor``, ``MXFP4Tensor`` with the same
``__slots__``) and ``ValueError`` messages as ``src/scratch_llm/quant/nvfp4_mxfp4.py`` (cited per
function), computed by the HIP kernels of ``libsqx_hip.so`` on ROCm device tensors and bit-identical
to the reference: codes, block scales and global scale. CPU tensors raise ``RuntimeError``.

Beyond the reference API, :func:`mxfp4_linear` and :func:`nvfp4_linear` run the linear on a
quantized weight without materialising it (``F.linear(x, dequant(W).to(x.dtype))``),
and :func:`quant_linear_nvfp4` keeps the reference's signature. Config 4's MXFP4-activation variant
(``mxfp4_linear(..., quantize_activations=True)``) quantizes the activation rows into the same tiled
layout (:func:`mxfp4_quantize_tiled`) and multiplies on CDNA4's block-scaled fp4 MFMA
(:func:`mxfp4_gemm`); at a few bf16 rows it streams the weight through the FP4 GEMV with the
dequantized activation rows instead (:func:`mxfp4_fake_quant_rows`, exact in bf16).
"""

from __future__ import annotations

import torch
from torch import Tensor

from scratch_llm_amd import _lib
from scratch_llm_amd.quant import _device

__all__ = [
    "E4M3_MAX",
    "FP4_MAGNITUDES",
    "FP4Tiled",
    "MXFP4Tensor",
    "NVFP4Tensor",
    "block_mse",
    "e2m1_decode",
    "e2m1_round_to_code",
    "fp4_linear_tiled",
    "MXFP4_GROUP",
    "dequantize_mxfp4",
    "mxfp4_dequantize",
    "mxfp4_fake_quant_rows",
    "mxfp4_gemm",
    "mxfp4_pack_weight",
    "mxfp4_linear",
    "mxfp4_quantize",
    "mxfp4_quantize_tiled",
    "nvfp4_dequantize",
    "nvfp4_linear",
    "nvfp4_quantize",
    "pack_fp4",
    "quant_linear_nvfp4",
    "quantize_e4m3",
    "quantize_e8m0",
    "sqnr_db",
    "tile_fp4",
    "tile_mxfp4_packed",
    "unpack_fp4",
]

FP4_MAGNITUDES: tuple[float, ...] = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)
E4M3_MAX = 448.0
_TINY = 1e-30
# Activation rows from which the tiled FP4 linear switches from the streaming decode kernel to the
# prefill GEMM.
GEMM_MIN_M = 64


def _float_input(x: Tensor, fn: str) -> Tensor:
    _lib.require_device(x, fn=fn)
    if x.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        x = x.to(torch.float32)
    return x.contiguous()


def _stream(t: Tensor) -> int:
    return _lib.stream_ptr(t.device)


# --------------------------------------------------------------------------------------
# FP4 (E2M1) element codec + nibble packing (nvfp4_mxfp4.py:85-129)
# --------------------------------------------------------------------------------------
def e2m1_round_to_code(x: Tensor) -> Tensor:
    """Round a pre-scaled tensor to E2M1 codes (bit 3 sign, bits 2-0 magnitude index), uint8, same
    shape (nvfp4_mxfp4.py:85-98): nearest magnitude by fp32 distance, ties to the lower one."""
    xf = _float_input(x, "e2m1_round_to_code")
    out = torch.empty(xf.shape, dtype=torch.uint8, device=xf.device)
    with torch.cuda.device(xf.device):
        _lib.check(_lib.load().sqx_e2m1_round(xf.data_ptr(), _lib.sqx_dtype(xf.dtype), xf.numel(), out.data_ptr(),
                                              _stream(xf)), "e2m1_round_to_code")
    return out


def e2m1_decode(code: Tensor) -> Tensor:
    """Decode 4-bit E2M1 codes to fp32 (nvfp4_mxfp4.py:101-106)."""
    _lib.require_device(code, fn="e2m1_decode")
    c = code.to(torch.uint8).contiguous()
    out = torch.empty(c.shape, dtype=torch.float32, device=c.device)
    with torch.cuda.device(c.device):
        _lib.check(_lib.load().sqx_e2m1_decode(c.data_ptr(), c.numel(), out.data_ptr(), _stream(c)), "e2m1_decode")
    return out


def pack_fp4(codes: Tensor) -> Tensor:
    """Pack a flat tensor of 4-bit codes two per byte, even element in the low nibble; an odd length
    is padded with a zero code (nvfp4_mxfp4.py:109-120)."""
    _lib.require_device(codes, fn="pack_fp4")
    c = codes.to(torch.uint8).reshape(-1).contiguous()
    n = c.numel()
    out = torch.empty((n + 1) // 2, dtype=torch.uint8, device=c.device)
    with torch.cuda.device(c.device):
        _lib.check(_lib.load().sqx_fp4_pack(c.data_ptr(), n, out.data_ptr(), _stream(c)), "pack_fp4")
    return out


def unpack_fp4(packed: Tensor, n: int) -> Tensor:
    """Inverse of :func:`pack_fp4`: the first ``n`` codes (nvfp4_mxfp4.py:123-129)."""
    _lib.require_device(packed, fn="unpack_fp4")
    p = packed.to(torch.uint8).reshape(-1).contiguous()
    n = int(min(n, 2 * p.numel()))
    out = torch.empty(max(n, 0), dtype=torch.uint8, device=p.device)
    with torch.cuda.device(p.device):
        _lib.check(_lib.load().sqx_fp4_unpack(p.data_ptr(), max(n, 0), out.data_ptr(), _stream(p)), "unpack_fp4")
    return out


# --------------------------------------------------------------------------------------
# Scale codecs (nvfp4_mxfp4.py:135-159)
# --------------------------------------------------------------------------------------
def _scale_codec(v: Tensor, fn: str, name: str) -> Tensor:
    _lib.require_device(v, fn=name)
    vf = v.to(torch.float32).contiguous()
    out = torch.empty(vf.shape, dtype=torch.float32, device=vf.device)
    with torch.cuda.device(vf.device):
        _lib.check(getattr(_lib.load(), fn)(vf.data_ptr(), vf.numel(), out.data_ptr(), _stream(vf)), name)
    return out


def quantize_e4m3(v: Tensor) -> Tensor:
    """Round non-negative magnitudes to the nearest E4M3 value (bias 7, saturating at 448, half to
    even), fp32 (nvfp4_mxfp4.py:135-147)."""
    return _scale_codec(v, "sqx_quantize_e4m3", "quantize_e4m3")


def quantize_e8m0(v: Tensor) -> Tensor:
    """Round positive magnitudes to the nearest power of two, ``2**round(log2 v)`` (nvfp4_mxfp4.py:150-159)."""
    return _scale_codec(v, "sqx_quantize_e8m0", "quantize_e8m0")


# --------------------------------------------------------------------------------------
# NVFP4 / MXFP4 payloads (nvfp4_mxfp4.py:190-272)
# --------------------------------------------------------------------------------------
class NVFP4Tensor:
    """The NVFP4 payload: E2M1 codes + fp32 global scale + per-block E4M3 scales (nvfp4_mxfp4.py:190-209)."""

    __slots__ = ("block", "codes", "n", "s_block", "s_global", "shape")

    def __init__(self, codes: Tensor, s_global: Tensor, s_block: Tensor, shape: torch.Size, n: int, block: int) -> None:
        self.codes = codes  # (n_blocks, block) uint8
        self.s_global = s_global  # scalar fp32
        self.s_block = s_block  # (n_blocks,) fp32, E4M3-representable
        self.shape = shape
        self.n = n
        self.block = block


class MXFP4Tensor:
    """The MXFP4 payload: E2M1 codes + per-block E8M0 (power-of-two) scales (nvfp4_mxfp4.py:237-254)."""

    __slots__ = ("block", "codes", "n", "s_block", "shape")

    def __init__(self, codes: Tensor, s_block: Tensor, shape: torch.Size, n: int, block: int) -> None:
        self.codes = codes
        self.s_block = s_block  # (n_blocks,) power-of-two
        self.shape = shape
        self.n = n
        self.block = block


def nvfp4_quantize(x: Tensor, block: int = 16) -> NVFP4Tensor:
    """Quantize ``x`` to NVFP4 (nvfp4_mxfp4.py:212-223): ``s_global = max(amax/2688, 1e-30)``,
    ``s_block = E4M3(block_amax / 6 / s_global)``, codes of ``x / (s_global * s_block)``."""
    xf = _float_input(x, "nvfp4_quantize")
    n = xf.numel()
    nb = -(-n // block)
    lib = _lib.load()
    codes = torch.empty(nb, block, dtype=torch.uint8, device=xf.device)
    s_block = torch.empty(nb, dtype=torch.float32, device=xf.device)
    s_global = torch.empty((), dtype=torch.float32, device=xf.device)
    ws = torch.empty(lib.sqx_nvfp4_workspace_bytes() // 4, dtype=torch.float32, device=xf.device)
    with torch.cuda.device(xf.device):
        _lib.check(lib.sqx_nvfp4_quantize(xf.data_ptr(), _lib.sqx_dtype(xf.dtype), n, block, codes.data_ptr(),
                                          s_block.data_ptr(), s_global.data_ptr(), ws.data_ptr(), ws.numel() * 4,
                                          _stream(xf)), "nvfp4_quantize")
    return NVFP4Tensor(codes, s_global, s_block, xf.shape, n, block)


def nvfp4_dequantize(q: NVFP4Tensor) -> Tensor:
    """Dequantize to fp32 in the original shape (nvfp4_mxfp4.py:226-231)."""
    _lib.require_device(q.codes, q.s_block, q.s_global, fn="nvfp4_dequantize")
    codes = q.codes.to(torch.uint8).contiguous()
    sb = q.s_block.to(torch.float32).contiguous()
    sg = q.s_global.to(torch.float32).reshape(()).contiguous()
    out = torch.empty(q.n, dtype=torch.float32, device=codes.device)
    with torch.cuda.device(codes.device):
        _lib.check(_lib.load().sqx_nvfp4_dequantize(codes.data_ptr(), sb.data_ptr(), sg.data_ptr(), q.n, q.block,
                                                    out.data_ptr(), _stream(codes)), "nvfp4_dequantize")
    return out.reshape(q.shape)


def mxfp4_quantize(x: Tensor, block: int = 32) -> MXFP4Tensor:
    """Quantize ``x`` to MXFP4 (nvfp4_mxfp4.py:257-265): no-overflow E8M0 block scale
    ``2**ceil(log2(max(amax/6, 1e-30)))`` and the E2M1 codes of ``x / s_block``."""
    xf = _float_input(x, "mxfp4_quantize")
    n = xf.numel()
    nb = -(-n // block)
    codes = torch.empty(nb, block, dtype=torch.uint8, device=xf.device)
    s_block = torch.empty(nb, dtype=torch.float32, device=xf.device)
    with torch.cuda.device(xf.device):
        _lib.check(_lib.load().sqx_mxfp4_quantize(xf.data_ptr(), _lib.sqx_dtype(xf.dtype), n, block,
                                                  codes.data_ptr(), s_block.data_ptr(), None, _stream(xf)),
                   "mxfp4_quantize")
    return MXFP4Tensor(codes, s_block, xf.shape, n, block)


def mxfp4_dequantize(q: MXFP4Tensor) -> Tensor:
    """Dequantize to fp32 in the original shape (nvfp4_mxfp4.py:268-272)."""
    _lib.require_device(q.codes, q.s_block, fn="mxfp4_dequantize")
    codes = q.codes.to(torch.uint8).contiguous()
    sb = q.s_block.to(torch.float32).contiguous()
    out = torch.empty(q.n, dtype=torch.float32, device=codes.device)
    with torch.cuda.device(codes.device):
        _lib.check(_lib.load().sqx_mxfp4_dequantize(codes.data_ptr(), sb.data_ptr(), q.n, q.block, out.data_ptr(),
                                                    _stream(codes)), "mxfp4_dequantize")
    return out.reshape(q.shape)


# --------------------------------------------------------------------------------------
# Metrics (nvfp4_mxfp4.py:278-290), float math on whatever device the tensors are on
# --------------------------------------------------------------------------------------
def sqnr_db(x: Tensor, x_hat: Tensor) -> float:
    """``10*log10(||x||^2 / ||x - x_hat||^2)`` in fp32, noise floored at 1e-30 (nvfp4_mxfp4.py:278-283)."""
    xf = x.to(torch.float32)
    sig = (xf**2).sum()
    noise = ((xf - x_hat.to(torch.float32)) ** 2).sum().clamp_min(_TINY)
    return float(10.0 * torch.log10(sig / noise))


def block_mse(x: Tensor, x_hat: Tensor, block: int) -> Tensor:
    """Per-block mean squared error over blocks of the flattened, zero-padded tensors (nvfp4_mxfp4.py:286-290)."""
    a = x.to(torch.float32).reshape(-1)
    b = x_hat.to(torch.float32).reshape(-1)
    pad = (-a.numel()) % block
    if pad:
        a = torch.nn.functional.pad(a, (0, pad))
        b = torch.nn.functional.pad(b, (0, pad))
    return ((a - b) ** 2).reshape(-1, block).mean(dim=1)


# --------------------------------------------------------------------------------------
# Linears on quantized weights
# --------------------------------------------------------------------------------------
class FP4Tiled:
    """An FP4 weight ``[rows, cols]`` re-laid for the linear kernels: ``wt`` (1 KiB per 16-row x
    128-column block), ``st`` (scale bytes), ``fmt`` (``_lib.FP4_MX`` or ``_lib.FP4_NV``) and the
    NVFP4 global scale as a device fp32 scalar (None for MXFP4)."""

    __slots__ = ("cols", "fmt", "rows", "s_global", "st", "wt")

    def __init__(self, wt: Tensor, st: Tensor, fmt: int, s_global: Tensor | None, rows: int, cols: int) -> None:
        self.wt, self.st, self.fmt, self.s_global, self.rows, self.cols = wt, st, fmt, s_global, rows, cols


def _weight_shape(q) -> tuple[int, int]:
    if len(q.shape) != 2:
        raise ValueError(f"a linear needs a 2-D weight, got shape {tuple(q.shape)}")
    rows, cols = int(q.shape[0]), int(q.shape[1])
    if cols % q.block != 0:
        raise ValueError(f"K={cols} must be a multiple of block={q.block} for the block-scaled GEMM")
    return rows, cols


def tile_fp4(q: MXFP4Tensor | NVFP4Tensor) -> FP4Tiled:
    """Re-lay a quantized 2-D weight for :func:`fp4_linear_tiled` (MXFP4 blocks a multiple of 32,
    NVFP4 blocks a multiple of 16)."""
    rows, cols = _weight_shape(q)
    nv = isinstance(q, NVFP4Tensor)
    if q.block % (16 if nv else 32) != 0:
        raise ValueError(f"the FP4 linear takes {'NVFP4' if nv else 'MXFP4'} blocks that are a multiple of "
                         f"{16 if nv else 32}, got block={q.block}")
    _lib.require_device(q.codes, q.s_block, fn="tile_fp4")
    lib = _lib.load()
    fmt = _lib.FP4_NV if nv else _lib.FP4_MX
    codes = q.codes.to(torch.uint8).contiguous()
    sb = q.s_block.to(torch.float32).contiguous()
    wt = torch.empty(lib.sqx_fp4_tiled_weight_bytes(rows, cols), dtype=torch.uint8, device=codes.device)
    st = torch.empty(lib.sqx_fp4_tiled_scale_bytes(rows, cols, fmt), dtype=torch.uint8, device=codes.device)
    kind = _lib.FP4_SCALE_NV_F32 if nv else _lib.FP4_SCALE_MX_F32
    with torch.cuda.device(codes.device):
        _lib.check(lib.sqx_fp4_tile(codes.data_ptr(), 0, sb.data_ptr(), kind, q.block, rows, cols, wt.data_ptr(),
                                    st.data_ptr(), _stream(codes)), "tile_fp4")
    s_global = q.s_global.to(torch.float32).reshape(()).contiguous() if nv else None
    return FP4Tiled(wt, st, fmt, s_global, rows, cols)


def untile_fp4(tw: FP4Tiled) -> tuple[Tensor, Tensor]:
    """A tiled FP4 weight back in the reference's byte form (``sqx_fp4_untile``, the exact inverse of
    the tilers): ``packed`` uint8 ``[out, in/2]`` in ``pack_fp4`` order (for MXFP4 the on-disk
    ``weight_packed``) and the scale bytes, E8M0 ``[out, in/32]`` (MXFP4, the on-disk ``weight_scale``)
    or E4M3 ``[out, in/16]`` (NVFP4, one per 16 columns)."""
    dev = _lib.require_device(tw.wt, tw.st, fn="untile_fp4")
    bs = 16 if tw.fmt == _lib.FP4_NV else 32
    packed = torch.empty(tw.rows, tw.cols // 2, dtype=torch.uint8, device=dev)
    scales = torch.empty(tw.rows, tw.cols // bs, dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        _lib.check(_lib.load().sqx_fp4_untile(tw.wt.data_ptr(), tw.st.data_ptr(), tw.fmt, tw.rows, tw.cols,
                                              packed.data_ptr(), scales.data_ptr(), _lib.stream_ptr(dev)), "untile_fp4")
    return packed, scales


def e4m3_values(codes: Tensor) -> Tensor:
    """fp32 values of E4M3 bytes (every one exact in fp32), through the FP8 row decoder at scale 1."""
    dev = _lib.require_device(codes, fn="e4m3_values")
    c = codes.to(torch.uint8).reshape(1, -1).contiguous()
    one = torch.ones(1, dtype=torch.float32, device=dev)
    out = torch.empty(c.shape[1], dtype=torch.float32, device=dev)
    if c.shape[1]:
        with torch.cuda.device(dev):
            _lib.check(_lib.load().sqx_fp8_dequantize_rows(c.data_ptr(), one.data_ptr(), 1, c.shape[1], out.data_ptr(),
                                                           _lib.stream_ptr(dev)), "e4m3_values")
    return out.reshape(codes.shape)


def fp4_linear_tiled(x: Tensor, tw: FP4Tiled, bias: Tensor | None = None, out_dtype: torch.dtype | None = None,
                     k_slices: int | None = None) -> Tensor:
    """``x @ W.T (+ bias)`` for a tiled FP4 weight. ``x`` is ``[..., cols]``: bf16 / fp16 run as they
    are; fp32 runs as two bf16 rows ``hi = bf16(x)``, ``lo = bf16(x - hi)`` through one pass over the
    weight (about 16 significant bits of x). The result is ``out_dtype`` (default: ``x.dtype``)."""
    *batch, k = x.shape
    if k != tw.cols:
        raise ValueError(f"x has in_features={k}, weight expects {tw.cols}")
    dev = _lib.require_device(x, tw.wt, bias, fn="fp4_linear")
    out_dtype = out_dtype or x.dtype
    lib = _lib.load()
    ks = 0 if k_slices is None else int(k_slices)
    x2 = x.reshape(-1, k)
    m = x2.shape[0]
    with torch.cuda.device(dev):
        s = _stream(x2)
        if x.dtype == torch.float32:
            if bias is not None:
                raise ValueError("fp32 activations take no bias in the FP4 linear")
            xf = x2.contiguous()
            xs = torch.empty(2 * m, k, dtype=torch.bfloat16, device=dev)
            _lib.check(lib.sqx_split_bf16(xf.data_ptr(), m * k, xs.data_ptr(), xs[m:].data_ptr(), s), "fp4_linear")
            y2 = torch.empty(2 * m, tw.rows, dtype=torch.float32, device=dev)
            if 2 * m >= GEMM_MIN_M and k_slices is None:
                ws = _lib.gemm_workspace(2 * m, tw.rows, tw.cols, dev)
                _lib.check(lib.sqx_fp4_gemm(tw.wt.data_ptr(), tw.st.data_ptr(), tw.fmt, _lib.ptr(tw.s_global), xs.data_ptr(),
                                            _lib.DTYPE_BF16, y2.data_ptr(), _lib.DTYPE_F32, None, 2 * m, tw.rows, tw.cols,
                                            *_lib.ws_args(ws), s), "fp4_linear")
            else:
                _lib.check(lib.sqx_fp4_linear(tw.wt.data_ptr(), tw.st.data_ptr(), tw.fmt, _lib.ptr(tw.s_global),
                                              xs.data_ptr(), _lib.DTYPE_BF16, y2.data_ptr(), _lib.DTYPE_F32, None, 2 * m,
                                              tw.rows, tw.cols, ks, s), "fp4_linear")
            y = torch.empty(m, tw.rows, dtype=torch.float32, device=dev)
            _lib.check(lib.sqx_sum_halves(y2.data_ptr(), m * tw.rows, y.data_ptr(), s), "fp4_linear")
            return y.reshape(*batch, tw.rows).to(out_dtype)
        if x.dtype not in (torch.bfloat16, torch.float16):
            raise TypeError(f"the FP4 linear takes fp32, bf16 or fp16 activations, got {x.dtype}")
        if not x2.is_contiguous() or x2.data_ptr() % 16:
            x2 = x2.contiguous()
        yf32 = out_dtype == torch.float32
        y = torch.empty(m, tw.rows, dtype=torch.float32 if yf32 else x.dtype, device=dev)
        b = None if bias is None else bias.to(x.dtype).contiguous()
        if b is not None and yf32:
            raise ValueError("a bias needs the output in the activation dtype")
        ydt = _lib.DTYPE_F32 if yf32 else _lib.sqx_dtype(x.dtype)
        if m >= GEMM_MIN_M and k_slices is None:
            ws = _lib.gemm_workspace(m, tw.rows, tw.cols, dev)
            _lib.check(lib.sqx_fp4_gemm(tw.wt.data_ptr(), tw.st.data_ptr(), tw.fmt, _lib.ptr(tw.s_global), x2.data_ptr(),
                                        _lib.sqx_dtype(x.dtype), y.data_ptr(), ydt, _lib.ptr(b), m, tw.rows, tw.cols,
                                        *_lib.ws_args(ws), s), "fp4_linear")
        else:
            _lib.check(lib.sqx_fp4_linear(tw.wt.data_ptr(), tw.st.data_ptr(), tw.fmt, _lib.ptr(tw.s_global),
                                          x2.data_ptr(), _lib.sqx_dtype(x.dtype), y.data_ptr(), ydt, _lib.ptr(b), m,
                                          tw.rows, tw.cols, ks, s), "fp4_linear")
        return y.reshape(*batch, tw.rows).to(out_dtype)


_tiled_cache = _device.TensorKeyedCache()


def _tiled(q: MXFP4Tensor | NVFP4Tensor) -> FP4Tiled:
    keys = (q.codes, q.s_block) if isinstance(q, MXFP4Tensor) else (q.codes, q.s_block, q.s_global)
    return _tiled_cache.get(keys, (type(q).__name__, tuple(q.shape), q.block), lambda: tile_fp4(q))


# --------------------------------------------------------------------------------------
# The on-disk MXFP4 pair (compressed-tensors mxfp4-pack-quantized, k3/checkpoint.py:92-144)
# --------------------------------------------------------------------------------------
MXFP4_GROUP = 32
_E8M0_NAN = 0xFF


def _check_mxfp4_pair(weight_packed: Tensor, weight_scale: Tensor) -> tuple[int, int]:
    """The reference loader's checks (k3/checkpoint.py:124-137), same messages."""
    if weight_packed.dtype != torch.uint8 or weight_scale.dtype != torch.uint8:
        raise ValueError(f"MXFP4 halves must be uint8; got {weight_packed.dtype}, {weight_scale.dtype}")
    if weight_packed.ndim != 2:
        raise ValueError(f"weight_packed must be [out, in/2]; got {tuple(weight_packed.shape)}")
    rows, cols = int(weight_packed.shape[0]), 2 * int(weight_packed.shape[1])
    groups = cols // MXFP4_GROUP
    if cols % MXFP4_GROUP or tuple(weight_scale.shape) != (rows, groups):
        raise ValueError(
            f"weight_packed {tuple(weight_packed.shape)} encodes [{rows}, {cols}], which needs "
            f"in % {MXFP4_GROUP} == 0 and weight_scale [{rows}, {groups}]; "
            f"got weight_scale {tuple(weight_scale.shape)}"
        )
    if bool((weight_scale == _E8M0_NAN).any()):
        raise ValueError("E8M0 scale 0xFF is NaN; refusing to load")
    return rows, cols


def mxfp4_pack_weight(q: MXFP4Tensor) -> tuple[Tensor, Tensor]:
    """A 2-D MXFP4 weight (block 32) as the on-disk pair: ``weight_packed`` uint8 ``[out, in/2]`` (low
    nibble = even element, ``pack_fp4`` order) and ``weight_scale`` uint8 E8M0 ``[out, in/32]``, the
    exponent byte of each power-of-two block scale."""
    if len(q.shape) != 2 or q.block != MXFP4_GROUP or int(q.shape[1]) % MXFP4_GROUP:
        raise ValueError(f"the on-disk MXFP4 pair needs a 2-D weight with in % 32 == 0 and block 32, got "
                         f"shape {tuple(q.shape)} and block {q.block}")
    rows, cols = int(q.shape[0]), int(q.shape[1])
    packed = pack_fp4(q.codes.reshape(-1)).reshape(rows, cols // 2)
    # a normal power of two 2**e has exponent field e + 127 (scales are >= 2**-99, never subnormal)
    e8 = ((q.s_block.to(torch.float32).contiguous().view(torch.int32) >> 23) & 0xFF).to(torch.uint8)
    return packed, e8.reshape(rows, cols // MXFP4_GROUP)


def tile_mxfp4_packed(weight_packed: Tensor, weight_scale: Tensor) -> FP4Tiled:
    """The tiled layout of the linear kernels straight from the on-disk pair (no repack on the host)."""
    rows, cols = _check_mxfp4_pair(weight_packed, weight_scale)
    dev = _lib.require_device(weight_packed, weight_scale, fn="tile_mxfp4_packed")
    lib = _lib.load()
    wp, ws = weight_packed.contiguous(), weight_scale.contiguous()
    wt = torch.empty(lib.sqx_fp4_tiled_weight_bytes(rows, cols), dtype=torch.uint8, device=dev)
    st = torch.empty(lib.sqx_fp4_tiled_scale_bytes(rows, cols, _lib.FP4_MX), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        _lib.check(lib.sqx_fp4_tile(wp.data_ptr(), 1, ws.data_ptr(), _lib.FP4_SCALE_MX_E8M0, MXFP4_GROUP, rows, cols,
                                    wt.data_ptr(), st.data_ptr(), _stream(wp)), "tile_mxfp4_packed")
    return FP4Tiled(wt, st, _lib.FP4_MX, None, rows, cols)


def dequantize_mxfp4(weight_packed: Tensor, weight_scale: Tensor, *, dtype: torch.dtype = torch.float32) -> Tensor:
    """``w[r, c] = E2M1(code[r, c]) * 2**(weight_scale[r, c // 32] - 127)`` as ``[out, in]`` in ``dtype``
    (k3/checkpoint.py:92-144). ``dtype=float64``: one HIP kernel decodes straight into float64, where
    every value of every E8M0 code is exact (so nothing raises, as in the reference). Other dtypes: the
    E2M1 decode and the scaling run in the HIP kernels in fp32, where every value below 2**128 is exact
    (E8M0 code 0 is 2**-127, a subnormal); values that overflow fp32, and casts to ``dtype`` that change
    a value, raise ``ValueError`` as in the reference."""
    rows, cols = _check_mxfp4_pair(weight_packed, weight_scale)
    dev = _lib.require_device(weight_packed, weight_scale, fn="dequantize_mxfp4")
    if dtype == torch.float64:
        out = torch.empty(rows, cols, dtype=torch.float64, device=dev)
        with torch.cuda.device(dev):
            _lib.check(_lib.load().sqx_mxfp4_pair_dequantize_f64(
                weight_packed.contiguous().data_ptr(), weight_scale.contiguous().data_ptr(), rows, cols,
                out.data_ptr(), _stream(out)), "dequantize_mxfp4")
        return out
    codes = unpack_fp4(weight_packed.reshape(-1), rows * cols)
    b = weight_scale.reshape(-1).to(torch.int32)
    s_block = torch.where(b == 0, torch.full_like(b, 0x00400000), b << 23).view(torch.float32)
    q = MXFP4Tensor(codes.reshape(-1, MXFP4_GROUP), s_block, torch.Size((rows, cols)), rows * cols, MXFP4_GROUP)
    out = mxfp4_dequantize(q)
    if not bool(torch.isfinite(out).all()):
        raise ValueError(f"MXFP4 values are not exact in {dtype} (overflow or underflow)")
    if dtype == torch.float32:
        return out
    cast = out.to(dtype)
    if not torch.equal(cast.to(torch.float32), out):
        raise ValueError(f"MXFP4 values are not exact in {dtype} (overflow or underflow)")
    return cast


def mxfp4_quantize_tiled(x: Tensor) -> FP4Tiled:
    """``mxfp4_quantize`` (block 32) of each row of a 2-D ``x`` ``[m, k]`` (``k % 32 == 0``) written
    straight into the tiled layout: the activation operand of :func:`mxfp4_gemm`. Codes and scales
    are bit-identical to ``tile_fp4(mxfp4_quantize(x))``."""
    if x.dim() != 2:
        raise ValueError(f"expected 2-D activations [m, k], got shape {tuple(x.shape)}")
    m, k = int(x.shape[0]), int(x.shape[1])
    if k % 32 != 0:
        raise ValueError(f"K={k} must be a multiple of 32 for per-row MXFP4 activation blocks")
    dev = _lib.require_device(x, fn="mxfp4_quantize_tiled")
    xc = _float_input(x, "mxfp4_quantize_tiled")
    if not xc.is_contiguous() or xc.data_ptr() % 16:
        xc = xc.contiguous()
    lib = _lib.load()
    xt = torch.empty(lib.sqx_fp4_tiled_weight_bytes(m, k), dtype=torch.uint8, device=dev)
    xst = torch.empty(lib.sqx_fp4_tiled_scale_bytes(m, k, _lib.FP4_MX), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        _lib.check(lib.sqx_mxfp4_quantize_tiled(xc.data_ptr(), _lib.sqx_dtype(xc.dtype), m, k, xt.data_ptr(),
                                                xst.data_ptr(), _stream(xc)), "mxfp4_quantize_tiled")
    return FP4Tiled(xt, xst, _lib.FP4_MX, None, m, k)


def mxfp4_gemm(xq: FP4Tiled, tw: FP4Tiled, bias: Tensor | None = None,
               out_dtype: torch.dtype = torch.bfloat16, *, splits: int = 0) -> Tensor:
    """``X @ W.T (+ bias)`` for tiled MXFP4 activations ``xq`` ``[m, k]`` and a tiled MXFP4 weight
    ``tw`` ``[n, k]`` on the block-scaled fp4 MFMA (fp32 accumulation), ``[m, n]`` in ``out_dtype``
    (bf16, fp16 or fp32; a bias needs bf16 or fp16).

    ``splits`` > 1 splits the k range over that many workgroups per output tile, through an fp32
    workspace summed in split order (deterministic); 0 lets the library choose (it splits when the
    output tiles would leave CUs idle, i.e. small ``m``)."""
    if xq.fmt != _lib.FP4_MX or tw.fmt != _lib.FP4_MX:
        raise ValueError("mxfp4_gemm takes MXFP4 operands on both sides")
    if xq.cols != tw.cols:
        raise ValueError(f"activations have in_features={xq.cols}, weight expects {tw.cols}")
    if out_dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError(f"mxfp4_gemm writes bf16, fp16 or fp32, not {out_dtype}")
    dev = _lib.require_device(xq.wt, tw.wt, bias, fn="mxfp4_gemm")
    if bias is not None and out_dtype == torch.float32:
        raise ValueError("a bias needs a bf16 or fp16 output")
    b = None if bias is None else bias.to(out_dtype).contiguous()
    y = torch.empty(xq.rows, tw.rows, dtype=out_dtype, device=dev)
    lib = _lib.load()
    nws = lib.sqx_mxfp4_gemm_workspace_bytes(xq.rows, tw.rows, tw.cols, int(splits))
    ws = torch.empty(nws, dtype=torch.uint8, device=dev) if nws > 0 else None
    with torch.cuda.device(dev):
        _lib.check(lib.sqx_mxfp4_gemm_ws(xq.wt.data_ptr(), xq.st.data_ptr(), tw.wt.data_ptr(), tw.st.data_ptr(),
                                         y.data_ptr(), _lib.sqx_dtype(out_dtype), _lib.ptr(b), xq.rows, tw.rows,
                                         tw.cols, int(splits), _lib.ptr(ws), nws, _stream(y)), "mxfp4_gemm")
    return y


def mxfp4_linear(x: Tensor, q: MXFP4Tensor, bias: Tensor | None = None, quantize_activations: bool = False) -> Tensor:
    """``F.linear(x, mxfp4_dequantize(q).to(x.dtype), bias)`` for an MXFP4 weight ``[out, in]``
    (BASELINE config 4's composition), without materialising the weight. Output in ``x.dtype``.

    ``quantize_activations=True`` is config 4's MXFP4-activation variant: each row of ``x`` goes
    through ``mxfp4_quantize`` too, and the product of the two dequantized operands is formed with
    exact products and fp32 accumulation: on the block-scaled fp4 MFMA GEMM, or, for bf16 ``x`` of at
    most ``MXFP4_ACT_GEMV_MAX_M`` rows, as the dequantized rows (exact in bf16,
    ``sqx_mxfp4_fake_quant_rows``) through the weight-streaming FP4 GEMV. It matches the composition
    with ``.to(x.dtype)`` wherever the dequantized values are representable in ``x.dtype`` (always
    for bf16 and fp32)."""
    tw = _tiled(q)
    if not quantize_activations:
        return fp4_linear_tiled(x, tw, bias)
    *batch, k = x.shape
    if k != tw.cols:
        raise ValueError(f"x has in_features={k}, weight expects {tw.cols}")
    if x.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise TypeError(f"the FP4 linear takes fp32, bf16 or fp16 activations, got {x.dtype}")
    x2 = x.reshape(-1, k)
    if x.dtype == torch.bfloat16 and x2.shape[0] <= MXFP4_ACT_GEMV_MAX_M:
        return fp4_linear_tiled(mxfp4_fake_quant_rows(x2), tw, bias).reshape(*batch, tw.rows)
    xq = mxfp4_quantize_tiled(x2)
    return mxfp4_gemm(xq, tw, bias, x.dtype).reshape(*batch, tw.rows)


# Rows up to which config 4's activation-quantized linear streams the weight through the FP4 GEMV
# instead of the 256-row fp4 MFMA GEMM (Llama-3-70B MLP shapes, rotating weights: at M = 1 the GEMV
# path takes 29.6 / 33.1 us against 64.1 / 43.5 us, at M = 2 37.5 / 44.5 against 63.3 / 43.6 us; from
# M = 4 the GEMM is as fast or faster).
MXFP4_ACT_GEMV_MAX_M = 2


def mxfp4_fake_quant_rows(x: Tensor) -> Tensor:
    """``mxfp4_dequantize(mxfp4_quantize(row))`` of each row of a 2-D ``x`` ``[m, k]`` (``k % 32 == 0``)
    as bf16 ``[m, k]``, exact (an E2M1 value times a power of two has 2 significant bits)."""
    if x.dim() != 2:
        raise ValueError(f"expected 2-D activations [m, k], got shape {tuple(x.shape)}")
    m, k = int(x.shape[0]), int(x.shape[1])
    if k % 32 != 0:
        raise ValueError(f"K={k} must be a multiple of 32 for per-row MXFP4 activation blocks")
    dev = _lib.require_device(x, fn="mxfp4_fake_quant_rows")
    xc = _float_input(x, "mxfp4_fake_quant_rows")
    if not xc.is_contiguous() or xc.data_ptr() % 16:
        xc = xc.contiguous()
    out = torch.empty(m, k, dtype=torch.bfloat16, device=dev)
    with torch.cuda.device(dev):
        _lib.check(_lib.load().sqx_mxfp4_fake_quant_rows(xc.data_ptr(), _lib.sqx_dtype(xc.dtype), m, k,
                                                         out.data_ptr(), _stream(xc)), "mxfp4_fake_quant_rows")
    return out


def nvfp4_linear(x: Tensor, q: NVFP4Tensor, bias: Tensor | None = None) -> Tensor:
    """``F.linear(x, nvfp4_dequantize(q).to(x.dtype), bias)`` for an NVFP4 weight ``[out, in]``."""
    return fp4_linear_tiled(x, _tiled(q), bias)


def quant_linear_nvfp4(x: Tensor, weight: Tensor, block: int = 16) -> Tensor:
    """Linear ``y = x @ weight.T`` with ``weight`` NVFP4-quantized along K (nvfp4_mxfp4.py:296-328):
    the weight is quantized on every call (shared global scale, E4M3 block scales) and the scales
    live inside the accumulation. ``x`` ``(M, K)`` in any float dtype; returns ``(M, N)`` fp32."""
    if weight.dim() != 2:
        raise ValueError(f"expected a 2-D weight, got shape {tuple(weight.shape)}")
    n_out, k = weight.shape
    if k % block != 0:
        raise ValueError(f"K={k} must be a multiple of block={block} for the block-scaled GEMM")
    if block % 16 != 0:
        raise ValueError(f"the NVFP4 linear kernels take blocks that are a multiple of 16, got block={block}")
    q = nvfp4_quantize(weight, block)
    tw = tile_fp4(q)
    return fp4_linear_tiled(x, tw, None, out_dtype=torch.float32)
