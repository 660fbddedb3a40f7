"""MXFP4 GEMMs with a fused output operation: the Triton ops of
aiter/ops/triton/gemm/fused/fused_gemm_afp4wfp4_{mul_add,split_cat,a16w16}.py,
served by this library's HIP GEMM kernels with the operation applied in their
epilogue (no intermediate product in HBM).

Layouts follow the reference ops:

* plain forms: ``x`` [M, K/2] and ``w`` [N, K/2] e2m1, scales [M, K/32] and
  [N, K/32] e8m0;
* preshuffled forms: ``w`` holds the ``shuffle_weight`` bytes (the Triton ops
  view them as [N/16, K*8]), ``w_scales`` the ``shuffle_scale`` bytes
  ([N/32, K]), and ``x_scales`` too when M >= 32 ([M/32, K]); for M < 32 the
  x scales are plain.

Only bf16 outputs are built (``dtype=torch.float16`` raises).  The Triton
tuning knobs (``config``, ``use_aot``) are accepted and unused; the GEMM
instance comes from this library's tuned table (preshuffled forms) or its
heuristic.  ``skip_reduce`` asks the reference for the split-K partials of a
split launch; this library never exposes partials and returns the finished
outputs, as the reference does for an unsplit launch.
"""
from __future__ import annotations

import torch
from torch import Tensor

from . import dtypes
from ._lib import call

__all__ = ["fused_gemm_afp4wfp4_mul_add", "fused_gemm_afp4wfp4_preshuffle_add_mul", "fused_gemm_afp4wfp4_split_cat",
           "fused_gemm_afp4wfp4_preshuffle_split_cat", "fused_gemm_afp4wfp4_a16w16"]


def _check_dtype(dtype):
    if dtype not in (None, dtypes.bf16):
        raise NotImplementedError(f"fused_gemm_afp4wfp4_*: only bf16 output is built (got {dtype})")


def _u8(t: Tensor) -> Tensor:
    return t.view(torch.uint8) if t.dtype != torch.uint8 else t


def _tuned_a4w4(m: int, n: int, k: int, preshuffled: bool) -> str | None:
    """The tuned A4W4 kernel of the shape when it names an instance of this
    library (the tuned table holds preshuffled-B rows only)."""
    if not preshuffled:
        return None
    from .gemm_op_a4w4 import _is_library_name, get_GEMM_config

    cfg = get_GEMM_config(m, n, k)
    name = str(cfg["kernelName"]) if cfg is not None else ""
    return name if name and _is_library_name(name) else None


def _operand(v, device):
    """(tensor or None, scalar) of a mul_add operand: Python numbers and
    host tensors of one element are scalars; device tensors are read in the
    epilogue (f32 or bf16; other float types are converted to f32)."""
    if isinstance(v, (int, float)):
        return None, float(v)
    if not isinstance(v, torch.Tensor):
        raise TypeError(f"mul_add operand must be a number or a tensor, got {type(v)}")
    if v.device.type != "cuda":
        if v.numel() != 1:
            raise ValueError("a host tensor operand must hold one element")
        return None, float(v.item())
    t = v if v.dtype in (torch.float32, dtypes.bf16) else v.float()
    if t.numel() != 1 and t.dim() == 1:
        t = t.view(1, -1)
    return t, 0.0


def _mul_add(x, w, x_scales, w_scales, a, b, y, fuse_type, preshuffled):
    m, k = x.shape[0], x.shape[1] * 2
    n = w.numel() * 2 // k if preshuffled else w.shape[0]
    if y is None:
        y = torch.empty((m, n), dtype=dtypes.bf16, device=x.device)
    ta, sa = _operand(a, x.device)
    tb, sb = _operand(b, x.device)
    call("fused_gemm_afp4wfp4_mul_add", _u8(x), _u8(w), _u8(x_scales), _u8(w_scales), ta, sa, tb, sb,
         int(fuse_type), y, int(preshuffled), _tuned_a4w4(m, n, k, preshuffled))
    return y


def fused_gemm_afp4wfp4_mul_add(x: Tensor, w: Tensor, x_scales: Tensor, w_scales: Tensor, a, b,
                                dtype: torch.dtype | None = dtypes.bf16, y: Tensor | None = None,
                                config: dict | None = None, fuse_type: int | None = 0) -> Tensor:
    """Y = a * (X W^T) + b (fuse_type 0) or a * b + X W^T (fuse_type 1), plain
    layouts (aiter/ops/triton/gemm/fused/fused_gemm_afp4wfp4_mul_add.py:63-236).
    ``a``/``b``: numbers, one-element tensors or tensors of the output shape."""
    _check_dtype(dtype)
    return _mul_add(x, w, x_scales, w_scales, a, b, y, fuse_type or 0, False)


def fused_gemm_afp4wfp4_preshuffle_add_mul(x: Tensor, w: Tensor, x_scales: Tensor, w_scales: Tensor, a, b,
                                           dtype: torch.dtype | None = dtypes.bf16, y: Tensor | None = None,
                                           config: dict | None = None, use_aot: bool | None = True,
                                           fuse_type: int | None = 0) -> Tensor:
    """The preshuffled-weight form of ``fused_gemm_afp4wfp4_mul_add``
    (fused_gemm_afp4wfp4_mul_add.py:239-)."""
    _check_dtype(dtype)
    return _mul_add(x, w, x_scales, w_scales, a, b, y, fuse_type or 0, True)


def _split_cat(x, w, y, x_scale, w_scale, S1, S2, preshuffled):
    m, k = x.shape[0], x.shape[1] * 2
    n = w.numel() * 2 // k if preshuffled else w.shape[0]
    mm, d, s3 = y.shape
    if mm != m or n != d * (S1 + S2):
        raise ValueError(f"N = {n} is not D * (S1 + S2) = {d} * ({S1} + {S2}), or y has {mm} rows for M = {m}")
    yy = y if y.dtype == dtypes.bf16 else y.to(dtypes.bf16)
    c1 = torch.empty((m, d, S1 + s3), dtype=dtypes.bf16, device=x.device)
    c2 = torch.empty((m, d, S2), dtype=dtypes.bf16, device=x.device)
    call("fused_gemm_afp4wfp4_split_cat", _u8(x), _u8(w), _u8(x_scale), _u8(w_scale), yy, c1, c2, int(S1), int(S2),
         int(preshuffled), _tuned_a4w4(m, n, k, preshuffled))
    return c1, c2


def fused_gemm_afp4wfp4_split_cat(x: Tensor, w: Tensor, y: Tensor, x_scale: Tensor, w_scale: Tensor, S1: int, S2: int,
                                  dtype: torch.dtype | None = dtypes.bf16, config: dict | None = None):
    """C = X W^T viewed [M, D, S1+S2], split into C1 = C[..., :S1] and C2 =
    C[..., S1:], then Y [M, D, S3] concatenated to C1: returns (c1 [M, D,
    S1+S3], c2 [M, D, S2]) (fused_gemm_afp4wfp4_split_cat.py:19-196).  S1, S2
    and S3 must be multiples of 8."""
    _check_dtype(dtype)
    return _split_cat(x, w, y, x_scale, w_scale, S1, S2, False)


def fused_gemm_afp4wfp4_preshuffle_split_cat(x: Tensor, w: Tensor, y: Tensor, x_scale: Tensor, w_scale: Tensor,
                                             S1: int, S2: int, dtype: torch.dtype | None = dtypes.bf16,
                                             config: dict | None = None):
    """The preshuffled-weight form (fused_gemm_afp4wfp4_split_cat.py:199-)."""
    _check_dtype(dtype)
    return _split_cat(x, w, y, x_scale, w_scale, S1, S2, True)


def fused_gemm_afp4wfp4_a16w16(x_fp4: Tensor, w_fp4: Tensor, x_fp4_scale: Tensor, w_fp4_scale: Tensor,
                               x_bf16: Tensor, w_bf16: Tensor, is_fp4_preshuffled: bool = True,
                               bias_fp4: Tensor | None = None, bias_bf16: Tensor | None = None,
                               dtype: float | None = dtypes.bf16, y_fp4: Tensor | None = None,
                               y_bf16: Tensor | None = None, skip_reduce: bool | None = False,
                               config: dict | None = None, use_aot: bool | None = True):
    """Y_fp4 = X_fp4 W_fp4^T (+ bias_fp4) and Y_bf16 = X_bf16 W_bf16^T
    (+ bias_bf16) over the same M and K (fused_gemm_afp4wfp4_a16w16.py:23-254):
    the gate-up projection and the MoE router of one layer in one call.
    Returns (y_fp4, y_bf16)."""
    _check_dtype(dtype)
    m, k = x_fp4.shape[0], x_fp4.shape[1] * 2
    if x_bf16.shape != (m, k):
        raise ValueError(f"x_bf16 must be [{m}, {k}] (same M and K as x_fp4), got {tuple(x_bf16.shape)}")
    n_fp4 = w_fp4.numel() * 2 // k if is_fp4_preshuffled else w_fp4.shape[0]
    n_bf16 = w_bf16.shape[0]
    if y_fp4 is None:
        y_fp4 = torch.empty((m, n_fp4), dtype=dtypes.bf16, device=x_fp4.device)
    if y_bf16 is None:
        y_bf16 = torch.empty((m, n_bf16), dtype=dtypes.bf16, device=x_bf16.device)
    b4 = None if bias_fp4 is None else bias_fp4.float().contiguous()
    b16 = None if bias_bf16 is None else bias_bf16.float().contiguous()
    from .tuned_gemm import get_GEMM_A16W16_config

    k4 = k16 = None
    if m > 64:
        # up to 64 rows the library runs both GEMMs in one grid (no kernel
        # names); above, each GEMM takes its tuned kernel, two launches
        cfg = get_GEMM_A16W16_config(m, n_bf16, k, bias_bf16 is not None, str(dtypes.bf16), str(dtypes.bf16))
        k16 = str(cfg.get("kernelName") or "") if cfg and cfg.get("libtype") == "aiter_amd" else ""
        k4 = _tuned_a4w4(m, n_fp4, k, is_fp4_preshuffled)
    call("fused_gemm_afp4wfp4_a16w16", _u8(x_fp4), _u8(w_fp4), _u8(x_fp4_scale), _u8(w_fp4_scale), b4, y_fp4,
         k4, x_bf16, w_bf16, b16, y_bf16, k16 or None, int(bool(is_fp4_preshuffled)))
    return y_fp4, y_bf16
