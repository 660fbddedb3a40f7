"""bf16 GEMM ctypes entry with the signature of aiter/ops/gemm_op_a16w16.py:61-76
(-> csrc/py_itfs_cu/asm_gemm_a16w16.cu:192-267).

The reference's split-K ASM kernels need a per-(device, stream) semaphore
workspace; this library's split-K path keeps its f32 partials in a
library-owned per-(device, stream) workspace, so the semaphore argument is an
empty tensor kept only for signature compatibility.
"""
from __future__ import annotations

import torch
from torch import Tensor

from ._lib import call

_SEMA_SHAPE = (16, 64)
ASM_SPLITK_MAX_GRID = _SEMA_SHAPE[0] * _SEMA_SHAPE[1]


def get_semaphore_workspace(device: torch.device) -> Tensor:
    return torch.empty((0,), dtype=torch.uint32, device=device)


def gemm_a16w16_asm(A: Tensor, B: Tensor, out: Tensor, bias: Tensor | None = None, splitK: int | None = None,
                    kernelName: str | None = None, bpreshuffle: bool = False):
    sema = get_semaphore_workspace(out.device)
    call("gemm_a16w16_asm", A, B, out, sema, bias, int(splitK) if splitK else 0, kernelName or None,
         int(bool(bpreshuffle)))
    return out
