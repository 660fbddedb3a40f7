"""Weight / scale layouts consumed by the GEMM kernels.

``shuffle_weight`` and ``shuffle_scale`` reproduce aiter's layouts
(aiter/ops/shuffle.py:148-209 and :339-365) as one-time torch permutations on
the tensor's own device.  The preshuffled weight is what makes every 16-row x
64-byte MFMA operand fragment a contiguous 1 KiB read in the kernels.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import dtypes


def shuffle_weight(x: torch.Tensor, layout=(16, 16), use_int4=False, pad_k_to: int = 0) -> torch.Tensor:
    """Preshuffle B (aiter/ops/shuffle.py:148-209, default non-MoE branch).

    View ``(-1, N/16, 16, Kel/BK, BK/Kp, Kp)`` and permute ``(0,1,3,4,2,5)``
    where ``Kp`` = 16 bytes worth of elements and ``BK = 2*layout[1]``.
    Sets ``is_shuffled = True`` on the result like the reference.
    """
    x_type = x.dtype
    if x_type in (dtypes.fp4x2, dtypes.fp8_e8m0) and x_type != torch.uint8:
        x = x.view(torch.uint8)
    original_k = x.shape[-1]
    if pad_k_to:
        if pad_k_to < 0:
            raise ValueError(f"shuffle_weight: pad_k_to is {pad_k_to}; it pads K up to a multiple and cannot be negative")
        padded = (original_k + pad_k_to - 1) // pad_k_to * pad_k_to
        if padded != original_k:
            x = F.pad(x.contiguous(), (0, padded - original_k), value=0)
    IN, IK = layout
    BK = IK * 2
    K = 16 // x.element_size() if not use_int4 else 32
    BN = IN
    assert x.shape[-2] % BN == 0, f"shuffle_weight: {x.shape[-2]} rows, not a whole number of {BN}-row blocks"
    assert x.shape[-1] % BK == 0, f"shuffle_weight: last dim {x.shape[-1]} is not a multiple of {BK}"
    x_ = x.view(-1, x.shape[-2] // BN, BN, x.shape[-1] // BK, BK // K, K)
    x_ = x_.permute(0, 1, 3, 4, 2, 5).contiguous()
    x_ = x_.view(*x.shape).view(x_type)
    x_.is_shuffled = True
    if pad_k_to:
        x_.aiter_original_k = original_k
        x_.aiter_padded_k = x.shape[-1]
    return x_


def shuffle_scale(src: torch.Tensor | None) -> torch.Tensor | None:
    """e8m0 scale swizzle (aiter/ops/shuffle.py:339-365, non-MoE branch):
    pad to (pad256(M), pad8(N)) and permute ``(M/32,2,16,N/8,2,4) ->
    (0,3,5,2,4,1)``.  f32 scales pass through unchanged."""
    if src is None:
        return src
    if src.dtype == torch.float32:
        return src
    assert src.ndim == 2, "scale must be a 2D tensor"
    m, n = src.shape
    padded = torch.zeros((m + 255) // 256 * 256, (n + 7) // 8 * 8, dtype=src.dtype, device=src.device)
    padded[:m, :n] = src
    sm, sn = padded.shape
    s = padded.view(sm // 32, 2, 16, sn // 8, 2, 4).permute(0, 3, 5, 2, 4, 1).contiguous()
    return s.view(sm, sn)


def e8m0_shuffle(scale):
    """Alias of ``shuffle_scale`` (aiter/utility/fp4_utils.py:224-227)."""
    return shuffle_scale(scale)
