"""Group-wise INT4 weights on MI355X — the API of ``scratch_llm.quant.int4_group``.

Same names, signatures, defaults, return types and ``ValueError`` messages as
``src/scratch_llm/quant/int4_group.py`` (cited per function), computed by the HIP kernels in
``libsqx_hip.so`` on ROCm device tensors. CPU tensors raise ``RuntimeError``: this module has no
host path.

Format (reference): signed codes in ``[-8, 7]``; ``scale = max(absmax(group) / 7, FLT_MIN)`` per
group of ``group_size`` consecutive input columns, fp32; packing puts the first element of a pair in
the high nibble. The linear itself runs on a tiled copy of the codes (:class:`Int4Tiled`), built
once per weight and cached for the functional entry point :func:`w4a16_linear`.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor

from scratch_llm_amd import _lib
from scratch_llm_amd.quant import _device

__all__ = [
    "GROUP_SIZE",
    "INT4_QMAX",
    "INT4_QMIN",
    "Int4Tiled",
    "dequantize_groupwise_int4",
    "int4_linear_tiled",
    "mse",
    "pack_int4",
    "quantize_groupwise_int4",
    "quantize_groupwise_uint4_asym",
    "sqnr_db",
    "tile_int4",
    "tile_int4_packed",
    "unpack_int4",
    "w4a16_linear",
]

GROUP_SIZE = 128
INT4_QMIN = -8
INT4_QMAX = 7

# Group sizes the tiled linear kernels take (a group never straddles a 32-column MFMA step).
TILED_GROUPS = (32, 64, 128)


# --------------------------------------------------------------------------- #
# Bit-exact nibble packing (int4_group.py:62-102)                              #
# --------------------------------------------------------------------------- #
def pack_int4(q: Tensor) -> Tensor:
    """Pack a 1-D signed 4-bit tensor into ``uint8``, two nibbles per byte (int4_group.py:62-82).

    The first element of each pair goes to the high nibble; an odd length gets a zero low nibble in
    the last byte. Returns ``uint8`` of length ``ceil(len(q) / 2)`` on ``q``'s device.
    """
    if q.dim() != 1:
        raise ValueError(f"pack_int4 expects a 1-D tensor, got shape {tuple(q.shape)}")
    dev = _lib.require_device(q, fn="pack_int4")
    n = q.numel()
    q8 = q.to(torch.int8).contiguous()  # keeps the low 4 bits of any integer code
    out = torch.empty((n + 1) // 2, dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        _lib.check(_lib.load().sqx_int4_pack(_lib.ptr(q8), n, _lib.ptr(out), _lib.stream_ptr(dev)), "pack_int4")
    return out


def unpack_int4(packed: Tensor, n: int) -> Tensor:
    """Inverse of :func:`pack_int4` (int4_group.py:85-102): high nibble first, sign-extended,
    the first ``n`` values as ``int8``."""
    if packed.dim() != 1:
        raise ValueError(f"unpack_int4 expects a 1-D tensor, got shape {tuple(packed.shape)}")
    dev = _lib.require_device(packed, fn="unpack_int4")
    n = int(min(n, 2 * packed.numel()))
    p8 = packed.to(torch.uint8).contiguous()
    out = torch.empty(max(n, 0), dtype=torch.int8, device=dev)
    with torch.cuda.device(dev):
        _lib.check(_lib.load().sqx_int4_unpack(_lib.ptr(p8), max(n, 0), _lib.ptr(out), _lib.stream_ptr(dev)),
                   "unpack_int4")
    return out


# --------------------------------------------------------------------------- #
# Group-wise symmetric INT4 quantizer (int4_group.py:108-142)                 #
# --------------------------------------------------------------------------- #
def quantize_groupwise_int4(w: Tensor, group_size: int = GROUP_SIZE) -> tuple[Tensor, Tensor]:
    """Symmetric group-wise INT4 quantization of a 2-D weight ``[out, in]`` (int4_group.py:108-129).

    Returns ``(q, scales)``: ``int8`` codes in ``[-8, 7]`` shaped like ``w`` and fp32 scales
    ``[out, in // group_size]``, bit-identical to the reference on the same input.
    """
    if w.dim() != 2:
        raise ValueError(f"expected a 2-D weight, got shape {tuple(w.shape)}")
    out_features, in_features = w.shape
    if in_features % group_size != 0:
        raise ValueError(f"in_features={in_features} not divisible by group_size={group_size}")
    dev = _lib.require_device(w, fn="quantize_groupwise_int4")
    if w.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        w = w.to(torch.float32)
    w = w.contiguous()
    q = torch.empty(out_features, in_features, dtype=torch.int8, device=dev)
    scales = torch.empty(out_features, in_features // group_size, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.load().sqx_int4_quantize_sym(
            _lib.ptr(w), _lib.sqx_dtype(w.dtype), out_features, in_features, group_size, _lib.ptr(q),
            _lib.ptr(scales), _lib.stream_ptr(dev),
        )
    _lib.check(rc, "quantize_groupwise_int4")
    return q, scales


def quantize_groupwise_uint4_asym(
    w: Tensor, group_size: int = GROUP_SIZE, param_dtype: torch.dtype = torch.bfloat16
) -> tuple[Tensor, Tensor, Tensor]:
    """Asymmetric group-wise uint4 (BASELINE config 2's format; no reference symbol — the 4-bit form
    of ``quantize_affine``, int8.py:142-172, per group of ``group_size`` input columns):
    ``lo = min(min(w), 0)``, ``hi = max(max(w), 0)``, ``s = max((hi - lo) / 15, 1e-12)`` rounded to
    ``param_dtype``, ``z = clamp(rint(-lo / s), 0, 15)``, ``q = clamp(rint(w / s + z), 0, 15)``.
    Returns ``(q uint8 [out, in], scales, zeros [out, in // group_size] of param_dtype)``; the
    dequantized weight is ``(q - z) * s``."""
    if w.dim() != 2:
        raise ValueError(f"expected a 2-D weight, got shape {tuple(w.shape)}")
    rows, cols = w.shape
    if cols % group_size != 0:
        raise ValueError(f"in_features={cols} not divisible by group_size={group_size}")
    if param_dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"param_dtype must be float32 or bfloat16, got {param_dtype}")
    dev = _lib.require_device(w, fn="quantize_groupwise_uint4_asym")
    wc = w.contiguous() if w.dtype in (torch.float32, torch.bfloat16, torch.float16) else w.float().contiguous()
    q = torch.empty(rows, cols, dtype=torch.uint8, device=dev)
    s = torch.empty(rows, cols // group_size, dtype=param_dtype, device=dev)
    z = torch.empty(rows, cols // group_size, dtype=param_dtype, device=dev)
    with torch.cuda.device(dev):
        _lib.check(_lib.load().sqx_int4_quantize_asym(wc.data_ptr(), _lib.sqx_dtype(wc.dtype), rows, cols, group_size,
                                                      _lib.sqx_dtype(param_dtype), q.data_ptr(), s.data_ptr(),
                                                      z.data_ptr(), _lib.stream_ptr(dev)),
                   "quantize_groupwise_uint4_asym")
    return q, s, z


def dequantize_groupwise_int4(q: Tensor, scales: Tensor, group_size: int = GROUP_SIZE) -> Tensor:
    """fp32 weights ``q * scale`` from INT4 codes and per-group scales (int4_group.py:132-142)."""
    out_features, in_features = q.shape
    dev = _lib.require_device(q, scales, fn="dequantize_groupwise_int4")
    q8 = q.to(torch.int8).contiguous()
    s32 = scales.to(torch.float32).contiguous()
    if s32.numel() != out_features * (in_features // group_size):
        raise ValueError(
            f"scales has {s32.numel()} elements, expected {out_features}x{in_features // group_size}"
        )
    out = torch.empty(out_features, in_features, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.load().sqx_int4_dequantize(
            _lib.ptr(q8), _lib.ptr(s32), out_features, in_features, group_size, _lib.ptr(out), _lib.stream_ptr(dev)
        )
    _lib.check(rc, "dequantize_groupwise_int4")
    return out


# --------------------------------------------------------------------------- #
# Tiled weights: the layout the linear kernels stream                          #
# --------------------------------------------------------------------------- #
@dataclass(frozen=True)
class Int4Tiled:
    """INT4 codes re-laid for the MI355X linear kernels.

    ``wt``: uint8, 1 KiB per (16-row tile, 128-column block); ``st``/``zt``: per-group scale and
    zero (``zt`` is None for symmetric codes) as ``[tiles][groups][16]``. Asymmetric codes with bf16
    parameters keep each (scale, zero) pair in one dword of ``st`` (``zt`` is then ``st`` itself, which
    marks the codes asymmetric). ``rows``/``cols`` are the logical weight shape ``[out, in]``.
    """

    wt: Tensor
    st: Tensor
    zt: Tensor | None
    rows: int
    cols: int
    group_size: int  # the kernels' group: 32, 64 or 128
    param_repeat: int = 1  # consecutive kernel groups that share one parameter of the source group

    @property
    def device(self) -> torch.device:
        return self.wt.device

    @property
    def nbytes(self) -> int:
        return self.wt.numel() + self.st.numel() * self.st.element_size() + (
            0 if self.zt is None or self.zt is self.st else self.zt.numel() * self.zt.element_size()
        )


def tiled_group(group_size: int) -> int:
    """The kernels' group (128, 64 or 32) for groups of ``group_size`` columns: the largest of them
    that divides it. A wider group (e.g. the reference tests' ``group_size = in_features``) runs as
    ``group_size // tiled_group`` kernel groups with its parameters repeated, so the dequantized
    weights are the same. ValueError for a group that is not a multiple of 32."""
    for g in (128, 64, 32):
        if group_size > 0 and group_size % g == 0:
            return g
    raise ValueError(f"group_size={group_size} is not supported by the tiled kernels (one of {TILED_GROUPS} "
                     "or a multiple of 32)")


def _check_tiled_group(group_size: int) -> None:
    tiled_group(group_size)


def _repeat_params(t: Tensor | None, rep: int) -> Tensor | None:
    return t if t is None or rep == 1 else t.repeat_interleave(rep, dim=1)


def tile_int4(
    q: Tensor, scales: Tensor, zeros: Tensor | None = None, group_size: int = GROUP_SIZE
) -> Int4Tiled:
    """Re-lay INT4 codes ``[out, in]`` and their group parameters for the linear kernels.

    Symmetric codes (``zeros is None``) are the reference's ``[-8, 7]`` codes with fp32 scales;
    asymmetric codes are unsigned ``[0, 15]`` with per-group ``scales`` and ``zeros`` (fp32 or bf16).
    """
    if q.dim() != 2:
        raise ValueError(f"expected 2-D codes, got shape {tuple(q.shape)}")
    rows, cols = q.shape
    if cols % group_size != 0:
        raise ValueError(f"in_features={cols} not divisible by group_size={group_size}")
    tg = tiled_group(group_size)
    rep = group_size // tg
    dev = _lib.require_device(q, scales, zeros, fn="tile_int4")
    pdt = torch.float32 if zeros is None else scales.dtype
    if pdt not in (torch.float32, torch.bfloat16):
        pdt = torch.float32
    s = _repeat_params(scales.to(pdt), rep).contiguous()
    z = None if zeros is None else _repeat_params(zeros.to(pdt), rep).contiguous()
    group_size = tg
    lib = _lib.load()
    wt = torch.empty(lib.sqx_int4_tiled_weight_bytes(rows, cols), dtype=torch.uint8, device=dev)
    npar = lib.sqx_int4_tiled_param_count(rows, cols, group_size)
    pairs = z is not None and pdt == torch.bfloat16  # (scale, zero) interleaved in st
    st = torch.empty(2 * npar if pairs else npar, dtype=pdt, device=dev)
    zt = None if z is None else (st if pairs else torch.empty(npar, dtype=pdt, device=dev))
    q8 = q.to(torch.int8).contiguous()
    with torch.cuda.device(dev):
        rc = lib.sqx_int4_tile(
            _lib.ptr(q8), 0 if z is None else 1, _lib.ptr(s), _lib.ptr(z), _lib.sqx_dtype(pdt), rows, cols,
            group_size, _lib.ptr(wt), _lib.ptr(st), _lib.ptr(zt), _lib.stream_ptr(dev),
        )
    _lib.check(rc, "tile_int4")
    return Int4Tiled(wt, st, zt, rows, cols, group_size, rep)


def tile_int4_packed(packed: Tensor, scales: Tensor, shape: tuple[int, int], group_size: int = GROUP_SIZE) -> Int4Tiled:
    """Re-lay the reference's packed byte stream (``pack_int4(q.reshape(-1))`` of symmetric codes of
    ``shape = (out, in)``) for the linear kernels, without unpacking it first."""
    rows, cols = shape
    if cols % group_size != 0:
        raise ValueError(f"in_features={cols} not divisible by group_size={group_size}")
    tg = tiled_group(group_size)
    rep = group_size // tg
    if packed.numel() != (rows * cols + 1) // 2:
        raise ValueError(f"packed has {packed.numel()} bytes, expected {(rows * cols + 1) // 2} for {shape}")
    dev = _lib.require_device(packed, scales, fn="tile_int4_packed")
    lib = _lib.load()
    p8 = packed.to(torch.uint8).contiguous()
    s = _repeat_params(scales.to(torch.float32), rep).contiguous()
    group_size = tg
    wt = torch.empty(lib.sqx_int4_tiled_weight_bytes(rows, cols), dtype=torch.uint8, device=dev)
    st = torch.empty(lib.sqx_int4_tiled_param_count(rows, cols, group_size), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = lib.sqx_int4_tile_packed(
            _lib.ptr(p8), _lib.ptr(s), _lib.DTYPE_F32, rows, cols, group_size, _lib.ptr(wt), _lib.ptr(st),
            _lib.stream_ptr(dev),
        )
    _lib.check(rc, "tile_int4_packed")
    return Int4Tiled(wt, st, None, rows, cols, group_size, rep)


def untile_int4(tw: Int4Tiled) -> tuple[Tensor, Tensor, Tensor | None]:
    """The reference's tensors back from a tiled weight (``sqx_int4_untile``, the exact inverse of the
    tilers): int8 codes ``[out, in]`` (signed ``[-8, 7]`` for symmetric weights, unsigned ``[0, 15]``
    when ``tw.zt`` is set), and the group scales (and zeros) ``[out, in/group]`` in the parameter dtype."""
    dev = _lib.require_device(tw.wt, tw.st, tw.zt, fn="untile_int4")
    lib = _lib.load()
    g = tw.cols // tw.group_size
    codes = torch.empty(tw.rows, tw.cols, dtype=torch.int8, device=dev)
    scales = torch.empty(tw.rows, g, dtype=tw.st.dtype, device=dev)
    zeros = None if tw.zt is None else torch.empty(tw.rows, g, dtype=tw.st.dtype, device=dev)
    with torch.cuda.device(dev):
        _lib.check(lib.sqx_int4_untile(tw.wt.data_ptr(), tw.st.data_ptr(), _lib.ptr(tw.zt), _lib.sqx_dtype(tw.st.dtype),
                                       0 if tw.zt is None else 1, tw.rows, tw.cols, tw.group_size, codes.data_ptr(),
                                       scales.data_ptr(), _lib.ptr(zeros), _lib.stream_ptr(dev)), "untile_int4")
    if tw.param_repeat > 1:  # one parameter per source group
        scales = scales[:, ::tw.param_repeat].contiguous()
        zeros = None if zeros is None else zeros[:, ::tw.param_repeat].contiguous()
    return codes, scales, zeros


# Activation rows from which the tiled linears switch from the decode-regime kernels (the streaming
# GEMV at one row; for 2..64 rows the library's choice among the GEMV and the row-tiled kernels, with
# K split into a workspace) to the prefill GEMM.
GEMM_MIN_M = 65


def int4_linear_tiled(x: Tensor, tw: Int4Tiled, bias: Tensor | None = None, k_slices: int | None = None) -> Tensor:
    """``x @ W.T (+ bias)`` for a tiled INT4 weight ``W [out, in]``; ``x`` is ``[..., in]`` in bf16 or
    fp16 and the result has ``x``'s dtype and shape ``[..., out]``. fp32 accumulation.

    With ``k_slices`` unset: one row runs the streaming decode GEMV; 2..``GEMM_MIN_M - 1`` rows the
    library's choice for the shape (the GEMV or a row-tiled decode kernel, K possibly split into a
    workspace, ``sqx_int4_skinny``); from ``GEMM_MIN_M`` rows on the prefill GEMM, which decodes each
    weight tile once per 256 rows to the reference's bf16 weights.

    ``k_slices`` (1..16) forces the decode GEMV with that many waves splitting each 16-row tile's
    columns. Every path adds its partial sums in a fixed order, so a call's bits depend only on the
    shape and ``k_slices``."""
    *batch, k = x.shape
    if k != tw.cols:
        raise ValueError(f"x has in_features={k}, weight expects {tw.cols}")
    dev = _lib.require_device(x, tw.wt, bias, fn="int4_linear_tiled")
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"int4_linear_tiled takes bf16 or fp16 activations, got {x.dtype}")
    x2 = x.reshape(-1, k)
    if not x2.is_contiguous() or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    m = x2.shape[0]
    y = torch.empty(m, tw.rows, dtype=x.dtype, device=dev)
    b = None if bias is None else bias.to(x.dtype).contiguous()
    lib = _lib.load()
    ks = 0 if k_slices is None else int(k_slices)
    with torch.cuda.device(dev):
        if 2 <= m < GEMM_MIN_M and k_slices is None:
            nb = int(lib.sqx_int4_skinny_workspace_bytes(m, tw.rows, tw.cols, 0))
            ws = torch.empty(nb // 4, dtype=torch.float32, device=dev) if nb > 0 else None
            rc = lib.sqx_int4_skinny(
                _lib.ptr(tw.wt), _lib.ptr(tw.st), _lib.ptr(tw.zt), _lib.sqx_dtype(tw.st.dtype), _lib.ptr(x2),
                _lib.sqx_dtype(x.dtype), _lib.ptr(y), _lib.ptr(b), m, tw.rows, tw.cols, tw.group_size, -1, 0, 0, 0,
                *_lib.ws_args(ws), _lib.stream_ptr(dev),
            )
        elif m >= GEMM_MIN_M and k_slices is None:
            ws = _lib.gemm_workspace(m, tw.rows, tw.cols, dev)
            rc = lib.sqx_int4_gemm(
                _lib.ptr(tw.wt), _lib.ptr(tw.st), _lib.ptr(tw.zt), _lib.sqx_dtype(tw.st.dtype), _lib.ptr(x2),
                _lib.sqx_dtype(x.dtype), _lib.ptr(y), _lib.ptr(b), m, tw.rows, tw.cols, tw.group_size,
                *_lib.ws_args(ws), _lib.stream_ptr(dev),
            )
        else:
            rc = lib.sqx_int4_linear(
                _lib.ptr(tw.wt), _lib.ptr(tw.st), _lib.ptr(tw.zt), _lib.sqx_dtype(tw.st.dtype), _lib.ptr(x2),
                _lib.sqx_dtype(x.dtype), _lib.ptr(y), _lib.ptr(b), m, tw.rows, tw.cols, tw.group_size, ks,
                _lib.stream_ptr(dev),
            )
    _lib.check(rc, "int4_linear_tiled")
    return y.reshape(*batch, tw.rows)


def int4_linear_skinny(
    x: Tensor, tw: Int4Tiled, bias: Tensor | None = None, *, variant: int = -1, tiles: int = 0, waves: int = 0,
    splits: int = 0,
) -> Tensor:
    """``x @ W.T (+ bias)`` for 1..64 rows of ``x`` on the decode-regime kernels with an explicit
    launch shape (``sqx_int4_skinny``): ``variant`` 0 = waves splitting K (``tiles`` 2 or 4 per wave,
    ``waves`` 1..8), 1 = activations staged through LDS (``tiles`` 1, 2 or 4 per wave, ``waves`` 4 or
    8 compute waves); ``splits`` workgroups along K (fp32 partials added in split order). -1 / 0
    pick the library's choice. A given shape always gives the same bits."""
    *batch, k = x.shape
    if k != tw.cols:
        raise ValueError(f"x has in_features={k}, weight expects {tw.cols}")
    dev = _lib.require_device(x, tw.wt, bias, fn="int4_linear_skinny")
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"int4_linear_skinny takes bf16 or fp16 activations, got {x.dtype}")
    x2 = x.reshape(-1, k)
    if not x2.is_contiguous() or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    m = x2.shape[0]
    if m > 64:
        raise ValueError(f"int4_linear_skinny takes at most 64 rows, got {m}")
    y = torch.empty(m, tw.rows, dtype=x.dtype, device=dev)
    b = None if bias is None else bias.to(x.dtype).contiguous()
    lib = _lib.load()
    nb = int(lib.sqx_int4_skinny_workspace_bytes(m, tw.rows, tw.cols, int(splits)))
    ws = torch.empty(nb // 4, dtype=torch.float32, device=dev) if nb > 0 else None
    with torch.cuda.device(dev):
        rc = lib.sqx_int4_skinny(
            _lib.ptr(tw.wt), _lib.ptr(tw.st), _lib.ptr(tw.zt), _lib.sqx_dtype(tw.st.dtype), _lib.ptr(x2),
            _lib.sqx_dtype(x.dtype), _lib.ptr(y), _lib.ptr(b), m, tw.rows, tw.cols, tw.group_size, int(variant),
            int(tiles), int(waves), int(splits), *_lib.ws_args(ws), _lib.stream_ptr(dev),
        )
    _lib.check(rc, "int4_linear_skinny")
    return y.reshape(*batch, tw.rows)


def int4_linear_tiled_f32(x: Tensor, tw: Int4Tiled, bias: Tensor | None = None,
                          col_scale: Tensor | None = None) -> Tensor:
    """``(x / col_scale) @ W.T (+ bias)`` for fp32 activations ``x [..., in]``, in fp32
    (``sqx_int4_linear_f32``): x splits into three bf16 rows whose sum is x exactly (8 significant
    bits each), which run through the int4 decode GEMV with fp32 outputs (exact code products, fp32
    group scales; 64 rows per pass over the weight) and are then added.
    ``col_scale`` is AWQ's per-input-channel scale (None: no division)."""
    *batch, k = x.shape
    if k != tw.cols:
        raise ValueError(f"x has in_features={k}, weight expects {tw.cols}")
    dev = _lib.require_device(x, tw.wt, bias, col_scale, fn="int4_linear_tiled_f32")
    if x.dtype != torch.float32:
        raise TypeError(f"int4_linear_tiled_f32 takes fp32 activations, got {x.dtype}")
    x2 = x.reshape(-1, k).contiguous()
    m = x2.shape[0]
    y = torch.empty(m, tw.rows, dtype=torch.float32, device=dev)
    b = None if bias is None else bias.to(torch.float32).contiguous()
    cs = None if col_scale is None else col_scale.to(torch.float32).contiguous()
    lib = _lib.load()
    nb = int(lib.sqx_int4_linear_f32_workspace_bytes(m, tw.rows, tw.cols))
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        rc = lib.sqx_int4_linear_f32(
            _lib.ptr(tw.wt), _lib.ptr(tw.st), _lib.ptr(tw.zt), _lib.sqx_dtype(tw.st.dtype), _lib.ptr(x2), _lib.ptr(cs),
            _lib.ptr(y), _lib.ptr(b), m, tw.rows, tw.cols, tw.group_size, ws.data_ptr(), nb, _lib.stream_ptr(dev),
        )
    _lib.check(rc, "int4_linear_tiled_f32")
    return y.reshape(*batch, tw.rows)


_tiled_cache = _device.TensorKeyedCache()


# --------------------------------------------------------------------------- #
# W4A16 linear (int4_group.py:148-164)                                         #
# --------------------------------------------------------------------------- #
def w4a16_linear(
    x: Tensor,
    q: Tensor,
    scales: Tensor,
    bias: Tensor | None = None,
    group_size: int = GROUP_SIZE,
) -> Tensor:
    """W4A16 linear (int4_group.py:148-164): ``x [..., in]`` times INT4 weights ``q/scales``
    describing ``[out, in]``; returns ``[..., out]`` in ``x``'s dtype.

    The fused dequant kernels run on a tiled copy of ``q`` that is built on first use and cached
    until ``q`` or ``scales`` changes. bf16/fp16 activations run as they are; fp32 activations run
    as three bf16 rows that sum to x exactly, with fp32 outputs (:func:`int4_linear_tiled_f32`).
    ``group_size`` must be a multiple of 32 (ValueError otherwise; a group wider than 128 runs as
    groups of 128, 64 or 32 with its scale repeated), and x must be fp32, bf16 or fp16 (TypeError
    otherwise).
    """
    _lib.require_device(x, q, scales, bias, fn="w4a16_linear")
    try:
        tiled_group(group_size)
    except ValueError:
        raise ValueError(f"w4a16_linear: group_size={group_size} is not supported by the MI355X kernels "
                         f"(one of {TILED_GROUPS} or a multiple of 32)") from None
    if x.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise TypeError(f"w4a16_linear takes fp32, bf16 or fp16 activations, got {x.dtype}")
    if q.shape[1] % group_size != 0:
        raise ValueError(f"in_features={q.shape[1]} not divisible by group_size={group_size}")
    tw = _tiled_cache.get((q, scales), (group_size,), lambda: tile_int4(q, scales, None, group_size))
    if x.dtype == torch.float32:
        return int4_linear_tiled_f32(x, tw, bias)
    return int4_linear_tiled(x, tw, bias)


# --------------------------------------------------------------------------- #
# Error metrics (int4_group.py:170-183)                                        #
# --------------------------------------------------------------------------- #
def sqnr_db(ref: Tensor, approx: Tensor) -> float:
    """Signal-to-quantization-noise ratio in dB: ``10*log10(P_signal/P_noise)`` (float64)."""
    ref = ref.to(torch.float64)
    approx = approx.to(torch.float64)
    signal = ref.pow(2).sum()
    noise = (ref - approx).pow(2).sum()
    if noise.item() == 0.0:
        return float("inf")
    return float(10.0 * torch.log10(signal / noise).item())


def mse(ref: Tensor, approx: Tensor) -> float:
    """Mean squared error between two tensors (float64 accumulation)."""
    return float((ref.to(torch.float64) - approx.to(torch.float64)).pow(2).mean().item())
