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


# ------------------------------------------------------ low-precision outputs
@torch.library.custom_op(f"{NS}::gemm_a4w4o4", mutates_args=(), device_types="cuda")
def gemm_a4w4o4(A: Tensor, B: Tensor, A_scale: Tensor, B_scale: Tensor) -> Tensor:
    from .gemm_op_a4w4 import gemm_a4w4o4 as op

    return op(A, B, A_scale, B_scale)


@gemm_a4w4o4.register_fake
def _(A, B, A_scale, B_scale):
    return A.new_empty((*A.shape[:-1], B.shape[0] // 2), dtype=dtypes.fp4x2)


@torch.library.custom_op(f"{NS}::gemm_a4w4o8", mutates_args=(), device_types="cuda")
def gemm_a4w4o8(A: Tensor, B: Tensor, A_scale: Tensor, B_scale: Tensor) -> Tuple[Tensor, Tensor]:
    from .gemm_op_a4w4 import gemm_a4w4o8 as op

    q, s = op(A, B, A_scale, B_scale)
    return q, s


@gemm_a4w4o8.register_fake
def _(A, B, A_scale, B_scale):
    n = B.shape[0]
    return (A.new_empty((*A.shape[:-1], n), dtype=dtypes.fp8),
            A.new_empty((*A.shape[:-1], n // 128), dtype=dtypes.fp8_e8m0))


# ------------------------------------------------------------- batched bf16
@torch.library.custom_op(f"{NS}::batched_gemm_bf16", mutates_args=(), device_types="cuda")
def batched_gemm_bf16(XQ: Tensor, WQ: Tensor, bias: Optional[Tensor] = None,
                      dtype: torch.dtype = dtypes.bf16) -> Tensor:
    from .batched_gemm_op_bf16 import batched_gemm_bf16_CK as op

    return op(XQ, WQ, bias, dtype)


@batched_gemm_bf16.register_fake
def _(XQ, WQ, bias=None, dtype=dtypes.bf16):
    return XQ.new_empty((XQ.shape[0], XQ.shape[1], WQ.shape[1]), dtype=dtype)


# --------------------------------------------------------------------- MoE
@torch.library.custom_op(f"{NS}::moe_sorting", mutates_args=(), device_types="cuda")
def moe_sorting(topk_ids: Tensor, topk_weights: Tensor, num_experts: int, model_dim: int,
                moebuf_dtype: torch.dtype = dtypes.bf16, block_size: int = 32
                ) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    from .fused_moe import moe_sorting as op

    return op(topk_ids, topk_weights, num_experts, model_dim, moebuf_dtype, block_size)


@moe_sorting.register_fake
def _(topk_ids, topk_weights, num_experts, model_dim, moebuf_dtype=dtypes.bf16, block_size=32):
    m, topk = topk_ids.shape
    padded = m * topk + num_experts * block_size - topk
    return (topk_ids.new_empty((padded,), dtype=torch.int32), topk_ids.new_empty((padded,), dtype=torch.float32),
            topk_ids.new_empty(((padded + block_size - 1) // block_size,), dtype=torch.int32),
            topk_ids.new_empty((2,), dtype=torch.int32), topk_ids.new_empty((m, model_dim), dtype=moebuf_dtype))


@torch.library.custom_op(f"{NS}::fused_moe", mutates_args=(), device_types="cuda")
def fused_moe(hidden_states: Tensor, w1: Tensor, w2: Tensor, topk_weight: Tensor, topk_ids: Tensor,
              w1_scale: Tensor, w2_scale: Tensor, expert_mask: Optional[Tensor] = None, activation: int = 0,
              doweight_stage1: bool = False, block_size_M: int = -1) -> Tensor:
    """QuantType.per_1x32 with MXFP4 weights (the schema keeps the arguments
    this library implements; see aiter_amd.fused_moe)."""
    from .fused_moe import ActivationType, fused_moe as op
    from .quant import QuantType

    return op(hidden_states, w1, w2, topk_weight, topk_ids, expert_mask=expert_mask,
              activation=ActivationType(activation), quant_type=QuantType.per_1x32,
              doweight_stage1=doweight_stage1, w1_scale=w1_scale, w2_scale=w2_scale,
              block_size_M=block_size_M if block_size_M > 0 else None)


@fused_moe.register_fake
def _(hidden_states, w1, w2, topk_weight, topk_ids, w1_scale, w2_scale, expert_mask=None, activation=0,
      doweight_stage1=False, block_size_M=-1):
    return hidden_states.new_empty((hidden_states.shape[0], w2.shape[1]), dtype=dtypes.bf16)


# ------------------------------------------------------- fused RMSNorm quant
@torch.library.custom_op(f"{NS}::fused_rms_mxfp4_quant", mutates_args=(), device_types="cuda")
def fused_rms_mxfp4_quant(x1: Tensor, x1_weight: Tensor, x1_epsilon: float,
                          shuffle: bool = False) -> Tuple[Tensor, Tensor]:
    """The single-input form of aiter_amd.fused_rms_mxfp4_quant: (fp4x2, e8m0)."""
    from .fused_quant import fused_rms_mxfp4_quant as op

    (q, s), _, _, _ = op(x1, x1_weight, x1_epsilon, shuffle=shuffle)
    return q, s


@fused_rms_mxfp4_quant.register_fake
def _(x1, x1_weight, x1_epsilon, shuffle=False):
    m, n = x1.shape
    sn = (n + 31) // 32
    shape = ((m + 255) // 256 * 256, (sn + 7) // 8 * 8) if shuffle else (m, sn)
    return x1.new_empty((m, n // 2), dtype=torch.uint8), x1.new_empty(shape, dtype=torch.uint8)


@torch.library.custom_op(f"{NS}::fused_rms_mxfp8_quant", mutates_args=(), device_types="cuda")
def fused_rms_mxfp8_quant(x: Tensor, weight: Tensor, eps: float) -> Tuple[Tensor, Tensor]:
    from .fused_quant import fused_rms_mxfp8_quant as op

    y, s = op(x, weight, eps)
    return y, s


@fused_rms_mxfp8_quant.register_fake
def _(x, weight, eps):
    m, k = x.shape
    return x.new_empty((m, k), dtype=dtypes.fp8), x.new_empty((m, k // 32), dtype=torch.uint8)


OPS = ("gemm_a4w4", "gemm_a4w4_asm", "gemm_a8w4_mxfp8", "gemm_a16w16", "gemm_a16w16_opus", "dynamic_mxfp4_quant",
       "dynamic_mxfp8_quant", "per_1x32_f4_quant_hip", "gemm_a4w4o4", "gemm_a4w4o8", "batched_gemm_bf16",
       "moe_sorting", "fused_moe", "fused_rms_mxfp4_quant", "fused_rms_mxfp8_quant")
