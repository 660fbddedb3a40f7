"""Batched bf16 GEMM (aiter/ops/batched_gemm_op_bf16.py): Y[b] = XQ[b] @ WQ[b]^T
(+ bias), one HIP launch over the batch (gridDim.z) on this library's bf16
tile kernels.

``batched_gemm_bf16`` / ``batched_gemm_bf16_tune`` keep the CK ops' argument
lists (:28-36, :127-134); ``batched_gemm_bf16_CK`` allocates the output as
the reference does (:104-124).  There is no tuned batched CSV here:
``get_CKBatchedGEMM_config`` returns None and the library's heuristic picks
the tile per (M, N, K).
"""
from __future__ import annotations

import torch
from torch import Tensor

from . import dtypes
from ._lib import call


def batched_gemm_bf16(XQ: Tensor, WQ: Tensor, out: Tensor, bias: Tensor | None = None, splitK: int = 0) -> Tensor:
    if bias is not None:
        bias = bias.float().contiguous()
    call("batched_gemm_bf16", XQ, WQ, out, bias, int(splitK))
    return out


def batched_gemm_bf16_tune(XQ: Tensor, WQ: Tensor, out: Tensor, kernelId: int, splitK: int = 0) -> Tensor:
    call("batched_gemm_bf16_tune", XQ, WQ, out, int(kernelId), int(splitK))
    return out


def compute_batched_gemm_SplitK(M: int, N: int, K: int, tile_m: int, tile_n: int, tile_k: int):
    """Kept for API parity (aiter/ops/batched_gemm_op_bf16.py:39-51); batched
    launches here run one pass over K."""
    return 0


def get_CKBatchedGEMM_config(B: int, M: int, N: int, K: int):
    return None


def batched_gemm_bf16_CK(XQ: Tensor, WQ: Tensor, bias: Tensor | None = None, dtype=dtypes.bf16,
                         splitK: int | None = None) -> Tensor:
    assert dtype in (dtypes.bf16, torch.float32), f"Output {dtype=} is not supported in batched_gemm_bf16"
    b, m, k = XQ.shape
    n = WQ.shape[1]
    Y = torch.empty(b, m, n, dtype=dtype, device=XQ.device)
    return batched_gemm_bf16(XQ, WQ, Y, bias, splitK or 0)
