"""The reference's CPU linear path restated with torch — TEST/BASELINE INFRASTRUCTURE ONLY.

scratch_llm computes every quantized linear by materialising the dequantized weight in fp32,
casting it to the activation dtype and calling ``torch.nn.functional.linear``
(int4_group.py:148-164, awq.py:184-192, nvfp4_mxfp4.py:268-272 composed with F.linear). This module
restates that composition on CPU tensors so ``bench.py`` can time it on the GPU box's host cores
beside the HIP kernels (``cpu_baseline``), and so tests can cross-check the numpy oracle.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def dequantize_groupwise_int4(q: torch.Tensor, scales: torch.Tensor, group_size: int = 128) -> torch.Tensor:
    """int4_group.py:132-142: fp32 codes times the group scale, [out, in] fp32."""
    rows, cols = q.shape
    g = cols // group_size
    return (q.to(torch.float32).view(rows, g, group_size) * scales.to(torch.float32).view(rows, g, 1)).view(rows, cols)


def w4a16_linear(x: torch.Tensor, q: torch.Tensor, scales: torch.Tensor, bias=None, group_size: int = 128):
    """int4_group.py:148-164: dequantize per call, cast to x's dtype, F.linear."""
    return F.linear(x, dequantize_groupwise_int4(q, scales, group_size).to(x.dtype), bias)


def int8_weight_linear(x: torch.Tensor, q: torch.Tensor, s: torch.Tensor, bias=None):
    """BASELINE config 1 (int8.py:127-129 composed with F.linear): x @ (q * s).to(x.dtype).T."""
    return F.linear(x, (q.to(torch.float32) * s.to(torch.float32).view(-1, 1)).to(x.dtype), bias)


_FP4 = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0])


def mxfp4_dequantize_packed(packed: torch.Tensor, e8m0: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    """nvfp4_mxfp4.py:123-129 + 268-272 on the packed form: low nibble = even element, value =
    E2M1(code) * 2**(e - 127) per 32-element block along a row."""
    lo = (packed & 0xF).long()
    hi = (packed >> 4).long()
    codes = torch.stack([lo, hi], dim=-1).reshape(rows, cols)
    vals = _FP4[codes]
    scale = torch.ldexp(torch.ones((), dtype=torch.float32), e8m0.to(torch.int32) - 127)
    return (vals.view(rows, cols // 32, 32) * scale.view(rows, cols // 32, 1)).view(rows, cols)


def mxfp4_linear(x: torch.Tensor, packed: torch.Tensor, e8m0: torch.Tensor, rows: int, cols: int, bias=None):
    """BASELINE config 4 oracle composition: F.linear(x, mxfp4_dequantize(W).to(x.dtype))."""
    return F.linear(x, mxfp4_dequantize_packed(packed, e8m0, rows, cols).to(x.dtype), bias)


def awq_linear(x: torch.Tensor, q: torch.Tensor, group_scales: torch.Tensor, chan_scale: torch.Tensor, bias=None,
               group_size: int = 128):
    """awq.py:178-192: W_eff = dequantize(q, group_scales) / chan_scale, cast to x's dtype, F.linear."""
    w = dequantize_groupwise_int4(q, group_scales, group_size) / chan_scale.to(torch.float32).view(1, -1)
    return F.linear(x, w.to(x.dtype), bias)
