"""Per-1x32 MX quantisers with the aiter Python signatures.

* ``per_1x32_mx_quant_hip`` / ``get_hip_quant(QuantType.per_1x32)``: the
  production RoundUp path (aiter/ops/quant.py:486-597 ->
  csrc/kernels/quant_kernels.cu:837-962).
* ``quant_mxfp4_hip``: the 4-round-mode quantiser (aiter/ops/quant.py:927-1033
  -> csrc/kernels/quant_mxfp4.cu:233-300).
* ``per_1x32_f4_quant_triton`` / ``get_triton_quant(QuantType.per_1x32)`` /
  ``dynamic_mxfp4_quant``: the Even-mode quant used by the A4W4 test and tuner
  (aiter/ops/quant.py:661-665 -> aiter/utility/fp4_utils.py:536-597), here a
  HIP kernel with the Triton kernel's byte layout.
* ``dynamic_mxfp8_quant``: Even-mode MXFP8 (aiter/ops/triton/quant/quant.py:235-297).

All of them run the HIP kernels of libaiter_amd.so.
"""
from __future__ import annotations

import enum
import functools

import torch

from . import dtypes
from ._lib import call


class QuantType(enum.IntEnum):
    """csrc/include/aiter_enum.h:17-27"""

    No = 0
    per_Tensor = 1
    per_Token = 2
    per_1x32 = 3
    per_1x128 = 4
    per_128x128 = 5
    per_256x128 = 6
    per_1024x128 = 7


class MxScaleRoundMode(enum.IntEnum):
    """csrc/include/mx_quant_utils.h:32-47 / aiter/utility/mx_types.py:35-49"""

    RoundDown = 0
    RoundUp = 1
    Even = 2
    Ceil = 3


MX_DEFAULT_ROUND_MODE = MxScaleRoundMode.RoundUp


def _scale_shape(m: int, n: int, shuffle: bool):
    sn = (n + 31) // 32
    if shuffle:
        return ((m + 255) // 256 * 256, (sn + 7) // 8 * 8)
    return (m, sn)


def per_1x32_mx_quant_hip(x, scale=None, quant_dtype=dtypes.fp4x2, shuffle=False,
                          num_rows: torch.Tensor | None = None, num_rows_factor=1, scale_type=None):
    """1x32 MX dynamic quant, RoundUp e8m0 (aiter/ops/quant.py:486-597).

    fp4x2: returns ``(y [m, n/2] fp4x2, scale e8m0)``; fp8: ``(y [m, n] e4m3,
    scale)`` with an e8m0 scale (``scale_type`` must be e8m0 or None here:
    the fp32-scale variant is not part of the MX path).
    """
    m, n = x.shape
    assert n % 32 == 0, f"n={n} must be divisible by 32"
    if scale is not None:
        raise ValueError("unsupported: static per token quant")
    if quant_dtype == dtypes.fp4x2:
        if scale_type is not None and scale_type not in (dtypes.fp8_e8m0,):
            raise ValueError("per_1x32_mx_quant_hip: fp4x2 output requires e8m0 scale")
        out_cols = n // 2
    elif quant_dtype == dtypes.fp8:
        if scale_type not in (None, dtypes.fp8_e8m0):
            raise NotImplementedError("only the e8m0 scale layout of MXFP8 is implemented")
        out_cols = n
    else:
        raise ValueError(f"per_1x32_mx_quant_hip: unsupported quant_dtype {quant_dtype}")
    scale = torch.empty(_scale_shape(m, n, shuffle), dtype=torch.uint8, device=x.device).view(dtypes.fp8_e8m0)
    y = torch.empty(m, out_cols, dtype=quant_dtype, device=x.device)
    dynamic_per_group_scaled_quant(y, x, scale, 32, shuffle_scale=shuffle, num_rows=num_rows,
                                   num_rows_factor=num_rows_factor)
    return y, scale


def dynamic_per_group_scaled_quant(out, input, scales, group_size=32, shuffle_scale=True,
                                   num_rows: torch.Tensor | None = None, num_rows_factor=1):
    """C entry csrc/kernels/quant_kernels.cu:837-962 (pybind defaults of
    csrc/include/rocm_ops.hpp)."""
    call("dynamic_per_group_scaled_quant", out, input, scales, int(group_size), int(bool(shuffle_scale)),
         num_rows, int(num_rows_factor))


def per_1x32_f4_quant_hip(x, scale=None, quant_dtype=dtypes.fp4x2, shuffle=False, num_rows=None,
                          num_rows_factor=1):
    """Legacy fp4 wrapper kept by the reference (aiter/ops/quant.py:600-615)."""
    return per_1x32_mx_quant_hip(x, scale, quant_dtype, shuffle, num_rows, num_rows_factor)


def quant_mxfp4_hip(x: torch.Tensor, group_size: int = 32, round_mode=MX_DEFAULT_ROUND_MODE,
                    e8m0_shuffle: bool = False, a16w4_shuffle: bool = False, gate_up: bool = False,
                    shuffle_weight: bool = False):
    """4-mode MXFP4 quant (aiter/ops/quant.py:927-1033).  RoundUp without
    layout flags takes the production path like the reference (:999-1006)."""
    assert x.is_contiguous() and x.dim() == 2
    assert x.dtype in (torch.float16, torch.bfloat16)
    rows, cols = x.shape
    assert cols % group_size == 0
    try:
        mode = int(round_mode)
    except (TypeError, ValueError) as e:
        raise ValueError(f"quant_mxfp4_hip: invalid round_mode={round_mode!r}") from e
    if mode not in (0, 1, 2, 3):
        raise ValueError(f"quant_mxfp4_hip: round_mode must be 0..3, got {mode}")
    if a16w4_shuffle or gate_up:
        raise NotImplementedError("a16w4/gate_up layouts are MoE-only and not part of this library")
    if mode == MxScaleRoundMode.RoundUp and not shuffle_weight:
        return per_1x32_f4_quant_hip(x, shuffle=e8m0_shuffle)
    out_packed = torch.empty(rows, cols // 2, dtype=dtypes.fp4x2, device=x.device)
    out_scale = torch.empty(_scale_shape(rows, cols, e8m0_shuffle), dtype=torch.uint8,
                            device=x.device).view(dtypes.fp8_e8m0)
    call("quant_mxfp4", x, out_packed, out_scale, int(group_size), mode, int(e8m0_shuffle), 0, 0,
         int(shuffle_weight))
    return out_packed, out_scale


def dynamic_mxfp4_quant(x: torch.Tensor, scaling_mode: str = "even", shuffle: bool = False):
    """Even-mode MXFP4 quant with the Triton kernel's layout
    (aiter/utility/fp4_utils.py:536-597): scale buffer [pad256(M), pad8(K/32)]
    (rows pad32(M).. untouched) when ``shuffle``, else [M, K/32]."""
    if scaling_mode != "even":
        raise ValueError(f"unsupported scaling_mode {scaling_mode!r}")
    M, N = x.shape
    assert (N // 2) % 2 == 0
    x_fp4 = torch.empty((M, N // 2), dtype=torch.uint8, device=x.device)
    if shuffle:
        bs = torch.empty(((M + 255) // 256 * 256, ((N + 31) // 32 + 7) // 8 * 8), dtype=torch.uint8,
                         device=x.device)
    else:
        bs = torch.empty((M, (N + 31) // 32), dtype=torch.uint8, device=x.device)
    call("dynamic_mxfp4_quant", x, x_fp4, bs, int(shuffle))
    return x_fp4.view(dtypes.fp4x2), bs.view(dtypes.fp8_e8m0)


def per_1x32_f4_quant_triton(x, scale=None, quant_dtype=dtypes.fp4x2, shuffle=False):
    """aiter/ops/quant.py:661-665 (the Triton entry), served by the HIP kernel."""
    assert quant_dtype == dtypes.fp4x2
    y, scale = dynamic_mxfp4_quant(x, shuffle=shuffle)
    return y.view(quant_dtype), scale


def dynamic_mxfp8_quant(x: torch.Tensor, shuffle: bool = False):
    """Even-mode MXFP8 (aiter/ops/triton/quant/quant.py:235-297): returns
    (y [M,K] e4m3fn, scale [M,K/32] e8m0) or a shuffled scale when asked."""
    M, K = x.shape
    assert K % 32 == 0
    y = torch.empty((M, K), dtype=dtypes.fp8, device=x.device)
    s = torch.empty(_scale_shape(M, K, shuffle), dtype=torch.uint8, device=x.device)
    call("dynamic_mxfp8_quant", x, y, s, int(shuffle))
    return y, s.view(dtypes.fp8_e8m0)


@functools.lru_cache
def get_hip_quant(qType):
    """aiter/ops/quant.py:367-387 (only the MX entry is part of this library)."""
    tmp = {
        QuantType.No.value: lambda *a, **k: (a[0], None),
        QuantType.per_1x32.value: per_1x32_mx_quant_hip,
    }

    def raise_NotImplementedError(*a, **k):
        raise NotImplementedError(f"unsupported quant type {qType=}")

    return tmp.get(int(qType), raise_NotImplementedError)


@functools.lru_cache
def get_triton_quant(qType):
    """aiter/ops/quant.py:390-403 (per_1x32 -> Even-mode MXFP4)."""
    tmp = {
        QuantType.No.value: lambda *a, **k: (a[0], None),
        QuantType.per_1x32.value: per_1x32_f4_quant_triton,
    }

    def raise_NotImplementedError(*a, **k):
        raise NotImplementedError(f"unsupported quant type {qType=}")

    return tmp.get(int(qType), raise_NotImplementedError)
