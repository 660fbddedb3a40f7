"""Fused RMSNorm -> MX quant prologues, on one HIP kernel (fused_quant.hip).

Mirrors the reference's Triton entry points, same names, arguments and
return values:
  fused_rms_mxfp4_quant   aiter/ops/triton/quant/fused_mxfp4_quant.py:23-147
  fused_rms_mxfp8_quant   aiter/ops/triton/quant/fused_mxfp8_quant.py:22-76
"""
from __future__ import annotations

import torch

from . import dtypes
from ._lib import call

_BLOCK = 32


def _cdiv(a: int, b: int) -> int:
    return (a + b - 1) // b


def fused_rms_mxfp4_quant(x1: torch.Tensor, x1_weight: torch.Tensor, x1_epsilon: float,
                          x2: torch.Tensor | None = None, x2_weight: torch.Tensor | None = None,
                          x2_epsilon: float = 0.0, res1: torch.Tensor | None = None,
                          shuffle: bool | None = False, scale_shuffle_padding: bool | None = False,
                          output_unquantized_inp1=False):
    """1. x1 += res1 (stored as out_res1), 2. RMSNorm(x1), 3. RMSNorm(x2) if
    given, 4. MXFP4 quant of the normalised x1 (Even e8m0 scales).  Returns
    ((out1_fp4 [M, N1/2] u8, out1_bs u8), out1, out2, out_res1); out1_bs is
    [pad256(M), pad8(N1/32)] (shuffled when ``shuffle``, padding columns of
    each row = 127) when ``shuffle`` or ``scale_shuffle_padding``, else
    [M, N1/32]."""
    M, N1 = x1.shape
    assert N1 % 2 == 0
    out1_fp4 = torch.empty((M, N1 // 2), dtype=torch.uint8, device=x1.device)
    padded = bool(shuffle or scale_shuffle_padding)
    sn = _cdiv(N1, _BLOCK)
    bs_shape = (_cdiv(M, 256) * 256, _cdiv(sn, 8) * 8) if padded else (M, sn)
    out1_bs = torch.empty(bs_shape, dtype=torch.uint8, device=x1.device)
    out1 = torch.empty((M, N1), dtype=x1.dtype, device=x1.device) if output_unquantized_inp1 else None
    out_res1 = torch.empty((M, N1), dtype=x1.dtype, device=x1.device) if res1 is not None else None
    out2 = torch.empty((M, x2.shape[1]), dtype=x1.dtype, device=x1.device) if x2 is not None else None
    call("fused_rms_mx_quant", x1, x1_weight, float(x1_epsilon), x2, x2_weight, float(x2_epsilon), res1, out1_fp4,
         out1_bs, out1, out2, out_res1, int(bool(shuffle)), int(padded))
    return (out1_fp4, out1_bs), out1, out2, out_res1


def fused_rms_mxfp8_quant(x: torch.Tensor, weight: torch.Tensor, eps: float, y: torch.Tensor | None = None,
                          scale: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """RMSNorm + MXFP8 (1x32 e8m0, Even) quant: (y [M, K] e4m3fn, scale [M, K/32] u8)."""
    assert x.dim() == 2, f"x must be 2D, got {x.dim()}"
    M, K = x.shape
    assert weight.shape == (K,), f"weight shape {tuple(weight.shape)} != ({K},)"
    assert K % _BLOCK == 0
    if y is None:
        y = torch.empty((M, K), dtype=dtypes.fp8, device=x.device)
    if scale is None:
        scale = torch.empty((M, K // _BLOCK), dtype=torch.uint8, device=x.device)
    call("fused_rms_mx_quant", x, weight, float(eps), None, None, 0.0, None, y, scale, None, None, None, 0, 0)
    return y, scale
