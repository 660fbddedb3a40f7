"""The library's ops as torch custom operators: ``torch.ops.aiter_amd.<name>``.

The reference reaches its ops through ``torch.ops.aiter.<name>`` as well as
through the Python functions (aiter/jit/utils/torch_guard.py:351-358: one
schema per op, an implementation on the device dispatch key and a fake
implementation for tracing).  This module does the same in its own
namespace, so that ``torch.compile`` and ``torch.export`` see each GEMM and
quantiser as one opaque node whose output shapes and dtypes come from the
fake implementations below, without running a kernel.

Only the CUDA (HIP) key has an implementation: called with CPU tensors the
ops raise torch's "could not run ... with arguments from the 'CPU' backend"
error (there is no CPU fallback).  Schemas follow the Python functions, with
two adjustments that tracing needs: ``gemm_a4w4_asm`` returns nothing (it
writes ``out``; a custom op may not return an alias of an input), and
``gemm_a16w16`` takes the preshuffled-B flag as an argument instead of
reading the ``is_shuffled`` attribute of B.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

from . import dtypes

NS = "aiter_amd"


def _pad(x: int, m: int) -> int:
    return (x + m - 1) // m * m


def _scale_shape(rows: int, k: int, shuffle: bool):
    kb = (k + 31) // 32
    return (_pad(rows, 256), _pad(kb, 8)) if shuffle else (rows, kb)


# ------------------------------------------------------------------ GEMMs
@torch.library.custom_op(f"{NS}::gemm_a4w4", mutates_args=(), device_types="cuda")
def gemm_a4w4(A: Tensor, B: Tensor, A_scale: Tensor, B_scale: Tensor, bias: Optional[Tensor] = None,
              alpha: float = 1.0, beta: float = 0.0, bpreshuffle: bool = True) -> Tensor:
    from .gemm_op_a4w4 import gemm_a4w4 as op

    return op(A, B, A_scale, B_scale, bias=bias, alpha=alpha, beta=beta, bpreshuffle=bpreshuffle)


@gemm_a4w4.register_fake
def _(A, B, A_scale, B_scale, bias=None, alpha=1.0, beta=0.0, bpreshuffle=True):
    return A.new_empty((*A.shape[:-1], B.shape[0]), dtype=dtypes.bf16)


@torch.library.custom_op(f"{NS}::gemm_a4w4_asm", mutates_args=("out",), device_types="cuda")
def gemm_a4w4_asm(A: Tensor, B: Tensor, A_scale: Tensor, B_scale: Tensor, out: Tensor, kernelName: str = "",
                  bias: Optional[Tensor] = None, alpha: float = 1.0, beta: float = 0.0, bpreshuffle: bool = True,
                  log2_k_split: int = 0) -> None:
    from .gemm_op_a4w4 import gemm_a4w4_asm as op

    op(A, B, A_scale, B_scale, out, kernelName, bias, alpha, beta, bpreshuffle, log2_k_split)


@gemm_a4w4_asm.register_fake
def _(A, B, A_scale, B_scale, out, kernelName="", bias=None, alpha=1.0, beta=0.0, bpreshuffle=True,
      log2_k_split=0):
    return None


@torch.library.custom_op(f"{NS}::gemm_a8w4_mxfp8", mutates_args=(), device_types="cuda")
def gemm_a8w4_mxfp8(A: Tensor, B: Tensor, ScaleA: Tensor, ScaleB: Tensor, a_preshuffle: bool = True,
                    kernelName: str = "") -> Tensor:
    from .gemm_op_a8w4 import gemm_a8w4_mxfp8 as op

    return op(A, B, ScaleA, ScaleB, a_preshuffle=a_preshuffle, kernelName=kernelName)


@gemm_a8w4_mxfp8.register_fake
def _(A, B, ScaleA, ScaleB, a_preshuffle=True, kernelName=""):
    return A.new_empty((A.shape[0], B.shape[0]), dtype=dtypes.bf16)


@torch.library.custom_op(f"{NS}::gemm_a16w16", mutates_args=(), device_types="cuda")
def gemm_a16w16(A: Tensor, B: Tensor, bias: Optional[Tensor] = None, otype: Optional[torch.dtype] = None,
                bpreshuffle: bool = False) -> Tensor:
    from .tuned_gemm import gemm_a16w16 as op

    if bpreshuffle != bool(getattr(B, "is_shuffled", False)):
        B = B.view(B.shape)          # a fresh view carries the flag without touching the caller's tensor
        B.is_shuffled = bpreshuffle
    return op(A, B, bias=bias, otype=otype)


@gemm_a16w16.register_fake
def _(A, B, bias=None, otype=None, bpreshuffle=False):
    return A.new_empty((*A.shape[:-1], B.shape[0]), dtype=otype if otype is not None else A.dtype)


@torch.library.custom_op(f"{NS}::gemm_a16w16_opus", mutates_args=(), device_types="cuda")
def gemm_a16w16_opus(A: Tensor, B: Tensor, bias: Optional[Tensor] = None,
                     dtype: torch.dtype = dtypes.bf16) -> Tensor:
    from .opus import gemm_a16w16_opus as op

    return op(A, B, bias, dtype)


@gemm_a16w16_opus.register_fake
def _(A, B, bias=None, dtype=dtypes.bf16):
    return A.new_empty((*A.shape[:-1], B.shape[-2]), dtype=dtype)


# ------------------------------------------------------------- quantisers
@torch.library.custom_op(f"{NS}::dynamic_mxfp4_quant", mutates_args=(), device_types="cuda")
def dynamic_mxfp4_quant(x: Tensor, shuffle: bool = False) -> Tuple[Tensor, Tensor]:
    from .quant import dynamic_mxfp4_quant as op

    y, s = op(x, shuffle=shuffle)
    return y, s


@dynamic_mxfp4_quant.register_fake
def _(x, shuffle=False):
    m, k = x.shape
    return (x.new_empty((m, k // 2), dtype=dtypes.fp4x2),
            x.new_empty(_scale_shape(m, k, shuffle), dtype=dtypes.fp8_e8m0))


@torch.library.custom_op(f"{NS}::dynamic_mxfp8_quant", mutates_args=(), device_types="cuda")
def dynamic_mxfp8_quant(x: Tensor, shuffle: bool = False) -> Tuple[Tensor, Tensor]:
    from .quant import dynamic_mxfp8_quant as op

    y, s = op(x, shuffle=shuffle)
    return y, s


@dynamic_mxfp8_quant.register_fake
def _(x, shuffle=False):
    m, k = x.shape
    return x.new_empty((m, k), dtype=dtypes.fp8), x.new_empty(_scale_shape(m, k, shuffle), dtype=dtypes.fp8_e8m0)


@torch.library.custom_op(f"{NS}::per_1x32_f4_quant_hip", mutates_args=(), device_types="cuda")
def per_1x32_f4_quant_hip(x: Tensor, shuffle: bool = False) -> Tuple[Tensor, Tensor]:
    from .quant import per_1x32_f4_quant_hip as op

    y, s = op(x, shuffle=shuffle)
    return y, s


@per_1x32_f4_quant_hip.register_fake
def _(x, shuffle=False):
    m, k = x.shape
    return (x.new_empty((m, k // 2), dtype=dtypes.fp4x2),
            x.new_empty(_scale_shape(m, k, shuffle), dtype=dtypes.fp8_e8m0))


OPS = ("gemm_a4w4", "gemm_a4w4_asm", "gemm_a8w4_mxfp8", "gemm_a16w16", "gemm_a16w16_opus", "dynamic_mxfp4_quant",
       "dynamic_mxfp8_quant", "per_1x32_f4_quant_hip")
