"""opus a16w16 API (aiter/ops/opus/gemm_op_a16w16.py:88-551).

``gemm_a16w16_opus(A, B, bias, dtype, kernelId, splitK, out)`` takes bf16
A [b, M, K] (or [M, K]) and B [b, N, K] (or [N, K]) and returns
Y [b, M, N] = A @ B^T (+ bias [N] or [b, N]).  ``kernelId`` is a reference
opus kernel id (csrc/opus_gemm/opus_gemm_common.py:238-513), run on this
library's kernel of the same tile (or its heuristic choice where it has
none), with ``splitK`` the literal split count; None uses the heuristic.
"""
from __future__ import annotations

import torch
from torch import Tensor

from . import dtypes
from ._lib import call


def _validate_and_reshape(A: Tensor, B: Tensor, bias: Tensor | None):
    """Layout guards of aiter/ops/opus/gemm_op_a16w16.py:315-441."""
    if A.dtype != dtypes.bf16 or B.dtype != dtypes.bf16:
        raise TypeError("gemm_a16w16_opus expects bf16 A and B")
    squeeze = A.dim() == 2
    if A.dim() == 2:
        A = A.unsqueeze(0)
    if B.dim() == 2:
        B = B.unsqueeze(0).expand(A.shape[0], -1, -1) if A.shape[0] > 1 else B.unsqueeze(0)
    if A.dim() != 3 or B.dim() != 3:
        raise ValueError("A and B must be 2-D or 3-D")
    if A.shape[0] != B.shape[0] or A.shape[2] != B.shape[2]:
        raise ValueError(f"shape mismatch A{tuple(A.shape)} B{tuple(B.shape)}")
    if A.stride(-1) != 1:
        A = A.contiguous()
    if B.stride(-1) != 1:
        B = B.contiguous()
    if bias is not None:
        if bias.dim() == 1:
            if bias.shape[0] != B.shape[1]:
                raise ValueError("bias must be [N] or [batch, N]")
        elif bias.dim() == 2:
            if bias.shape != (A.shape[0], B.shape[1]):
                raise ValueError("bias must be [N] or [batch, N]")
        else:
            raise ValueError("bias must be [N] or [batch, N]")
        bias = bias.float().contiguous()
    return A, B, bias, squeeze


def opus_gemm_a16w16_tune(XQ: Tensor, WQ: Tensor, Y: Tensor, bias: Tensor | None = None, kernelId: int = 0,
                          splitK: int = 0) -> Tensor:
    """Explicit-kernel entry (csrc/opus_gemm/opus_gemm.cu:294-350).  ``splitK``
    is a literal split count (KBatch); 0 or 1 runs one pass.

    Older positional calls ``opus_gemm_a16w16_tune(XQ, WQ, Y, kernelId, splitK)``
    keep working as in aiter/ops/opus/gemm_op_a16w16.py:196-210: an int in the
    bias slot is the kernel id and the next positional int the split count."""
    if isinstance(bias, int) and not isinstance(bias, bool):
        new_split = splitK if (splitK != 0 and kernelId == 0) else kernelId
        kernelId, splitK, bias = bias, new_split, None
    call("opus_gemm_a16w16_tune", XQ, WQ, Y, bias, int(kernelId), int(splitK))
    return Y


def gemm_a16w16_opus(A: Tensor, B: Tensor, bias: Tensor | None = None, dtype: torch.dtype = dtypes.bf16, *,
                     kernelId: int | None = None, splitK: int | None = None, out: Tensor | None = None) -> Tensor:
    A3, B3, bias, squeeze = _validate_and_reshape(A, B, bias)
    b, M, _ = A3.shape
    N = B3.shape[1]
    if out is None:
        out = torch.empty((b, M, N), dtype=dtype, device=A.device)
    Y = out if out.dim() == 3 else out.view(b, M, N)
    if kernelId is not None:
        opus_gemm_a16w16_tune(A3, B3, Y, bias, int(kernelId), int(splitK or 0))
    else:
        call("opus_gemm", A3, B3, Y, bias)
    return Y[0] if squeeze and out.dim() == 3 else out


def opus_gemm_workspace_init(device=None, max_bytes: int = 64 << 20):
    """Pre-size the split-K workspace of the current stream so later calls can
    be graph-captured (the role of opus_gemm_workspace_init / the prewarm in
    aiter/tuned_gemm.py:54-137)."""
    from ._lib import lib

    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    st = torch.cuda.current_stream(dev).cuda_stream
    rc = lib().gemm_workspace_reserve(dev.index or 0, st, int(max_bytes))
    if rc != 0:
        raise RuntimeError(f"gemm_workspace_reserve failed: {lib().aiter_get_last_error()}")
