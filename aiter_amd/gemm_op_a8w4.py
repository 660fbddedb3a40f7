"""MXFP8 (activation) x MXFP4 (weight) GEMM with the signature of
aiter/ops/gemm_op_a8w4.py:34-61 (a gfx1250-only ASM op in the reference),
implemented for gfx950 with the scaled MFMA (A format e4m3, B format e2m1).

A [M, K] e4m3fn (row-major, or ``shuffle_weight`` layout when
``a_preshuffle``), B [N, K/2] fp4x2 preshuffled, ScaleA / ScaleB e8m0 in the
shuffled layout, output [M, N] bf16.  ``gemm_a8w4_mxfp8_dynamic`` adds the
fused dynamic activation quant from a bf16 input.
"""
from __future__ import annotations

import functools

import torch
from torch import Tensor

from . import dtypes
from ._lib import call
from .config import A4W4_KEYS, DEFAULT_A8W4_CSV, get_cu_num, get_gfx, load_tuned
from .gemm_common import get_padded_m
from .quant import per_1x32_mx_quant_hip, dynamic_mxfp8_quant
from .shuffle import shuffle_weight


@functools.lru_cache(maxsize=1)
def _a8w4_table():
    return load_tuned("AITER_CONFIG_GEMM_A8W4", DEFAULT_A8W4_CSV, A4W4_KEYS)


@functools.lru_cache(maxsize=1024)
def get_GEMM_A8W4_config(M: int, N: int, K: int):
    """Tuned row for (gfx, cu_num, M | padded M, N, K), same schema and
    padded-M retries as the A4W4 table (aiter/ops/gemm_op_a4w4.py:33-78)."""
    table = _a8w4_table()
    gfx, cu_num = get_gfx(), get_cu_num()
    for gl in (None, 0, 1):
        pm = M if gl is None else get_padded_m(M, N, K, gl)
        cfg = table.get((gfx, cu_num, pm, N, K))
        if cfg is not None:
            return cfg
    return None


def gemm_a8w4_mxfp8(A: Tensor, B: Tensor, ScaleA: Tensor, ScaleB: Tensor, dtype: torch.dtype = dtypes.bf16,
                    a_preshuffle: bool = True, kernelName: str = "") -> Tensor:
    if dtype != dtypes.bf16:
        raise NotImplementedError("gemm_a8w4_mxfp8 produces bf16 output")
    M = A.shape[0]
    N = B.shape[0]
    out = torch.empty((M, N), dtype=dtype, device=A.device)
    if not kernelName and not a_preshuffle:
        cfg = get_GEMM_A8W4_config(M, N, A.shape[1])
        if cfg is not None:
            kernelName = str(cfg["kernelName"])
    call("mxfp8_mxfp4_gemm_asm", A, B, ScaleA, ScaleB, out, kernelName if kernelName else None,
         int(bool(a_preshuffle)))
    return out


def gemm_a8w4_mxfp8_dynamic(x: Tensor, B: Tensor, ScaleB: Tensor, round_mode: str = "even",
                            kernelName: str = "") -> Tensor:
    """bf16 activation -> dynamic MXFP8 (e4m3 + shuffled e8m0) -> GEMM.
    ``round_mode`` "even" uses the Triton dynamic_mxfp8_quant rounding
    (aiter/ops/triton/quant/quant.py:235-297), "up" the HIP RoundUp path."""
    if round_mode == "even":
        a, sa = dynamic_mxfp8_quant(x, shuffle=True)
    elif round_mode == "up":
        a, sa = per_1x32_mx_quant_hip(x, quant_dtype=dtypes.fp8, shuffle=True, scale_type=dtypes.fp8_e8m0)
    else:
        raise ValueError(f"unknown round_mode {round_mode!r}")
    return gemm_a8w4_mxfp8(a, B, sa, ScaleB, a_preshuffle=False, kernelName=kernelName)
