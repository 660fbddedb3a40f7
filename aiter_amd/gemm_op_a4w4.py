"""MXFP4 x MXFP4 (A4W4) GEMM with aiter's Python API
(aiter/ops/gemm_op_a4w4.py:20-287, 581-608).

D[M, N] = (A (x) A_scale) @ (B (x) B_scale)^T, A [M, K/2] fp4x2 row-major,
B [N, K/2] fp4x2 preshuffled (``shuffle_weight``), both scales e8m0 in the
shuffled layout (``shuffle_scale``), output bf16 allocated as [pad32(M), N]
and returned as ``out[:M]`` like the reference.
"""
from __future__ import annotations

import functools
import logging
import os

import torch
from torch import Tensor

from . import dtypes
from ._lib import call
from .config import A4W4_KEYS, DEFAULT_A4W4_CSV, get_cu_num, get_gfx, load_tuned
from .gemm_common import get_padded_m

logger = logging.getLogger("aiter_amd")
AITER_LOG_TUNED_CONFIG = int(os.environ.get("AITER_LOG_TUNED_CONFIG", "0"))


@functools.lru_cache(maxsize=1024)
def compute_gemm_SplitK(M: int, N: int, K: int, tile_m: int, tile_n: int, tile_k: int):
    """Tuner's split-K upper bound; the reference returns 3 unconditionally
    (aiter/ops/gemm_op_a4w4.py:20-30)."""
    return 3


@functools.lru_cache(maxsize=1)
def _a4w4_table():
    return load_tuned("AITER_CONFIG_GEMM_A4W4", DEFAULT_A4W4_CSV, A4W4_KEYS)


@functools.lru_cache(maxsize=1024)
def get_GEMM_config(M: int, N: int, K: int):
    """CSV row for (gfx, cu_num, M | padded(M, gl=0) | padded(M, gl=1), N, K)
    (aiter/ops/gemm_op_a4w4.py:33-78)."""
    table = _a4w4_table()
    gfx, cu_num = get_gfx(), get_cu_num()
    for gl in (None, 0, 1):
        pm = M if gl is None else get_padded_m(M, N, K, gl)
        cfg = table.get((gfx, cu_num, pm, N, K))
        if cfg is not None:
            if AITER_LOG_TUNED_CONFIG:
                logger.info(f"shape M:{M} N:{N} K:{K} tuned as padded_M {pm}: {cfg['kernelName']}")
            return cfg
    logger.debug(f"shape M:{M} N:{N} K:{K} not tuned, using the heuristic")
    return None


def gemm_a4w4_fake(A, B, A_scale, B_scale, bias=None, dtype=dtypes.bf16, alpha=1.0, beta=0.0,
                   bpreshuffle=True, apreshuffle=False, global_A_scale=None, global_B_scale=None):
    n = B.shape[0]
    return torch.empty((*A.shape[:-1], n), dtype=dtype, device=A.device)


def gemm_a4w4(A: Tensor, B: Tensor, A_scale: Tensor, B_scale: Tensor, bias: Tensor | None = None,
              dtype: torch.dtype = dtypes.bf16, alpha: float | None = 1.0, beta: float | None = 0.0,
              bpreshuffle: bool | None = True, apreshuffle: bool | None = False,
              global_A_scale: Tensor | None = None, global_B_scale: Tensor | None = None) -> Tensor:
    """A4W4 GEMM (aiter/ops/gemm_op_a4w4.py:147-238).  NVFP4 global scales and
    low-precision outputs are gfx1250-only in the reference and rejected."""
    if dtype in (dtypes.fp4x2, dtypes.fp8):
        raise NotImplementedError("gemm_a4w4 returns one plain-dtype tensor")
    if global_A_scale is not None or global_B_scale is not None:
        raise NotImplementedError("NVFP4 global scales are a gfx1250 feature")
    if apreshuffle:
        raise NotImplementedError("preshuffled A is a gfx1250 feature of gemm_a4w4")
    if dtype != dtypes.bf16:
        raise NotImplementedError("gemm_a4w4 produces bf16 output")
    m = A.numel() // A.shape[-1]
    n = B.shape[0]
    out = torch.empty(((m + 31) // 32 * 32, n), dtype=dtype, device=A.device)
    _gemm_a4w4_into(A, B, A_scale, B_scale, out, bias, alpha, beta, bpreshuffle)
    return out[:m].view(*A.shape[:-1], n)


def _gemm_a4w4_into(A: Tensor, B: Tensor, A_scale: Tensor, B_scale: Tensor, out: Tensor, bias: Tensor | None,
                    alpha, beta, bpreshuffle) -> None:
    """The tuned dispatch of gemm_a4w4 into a caller-given out [>= M, N] (the
    tests pass a NaN-filled one to see that every output tile is written)."""
    m = A.numel() // A.shape[-1]
    n = B.shape[0]
    k = A.shape[-1] * 2
    cfg = get_GEMM_config(m, n, k)
    split_k = 0
    kernel_name = ""
    if cfg is not None:
        split_k = int(cfg.get("splitK", 0) or 0)
        kernel_name = str(cfg["kernelName"])
        if kernel_name in _UNRESOLVED_NAMES:
            # served by the heuristic, with its own split choice, on every call
            # of the shape (the first call's fallback below does the same)
            kernel_name, split_k = "", 0
    try:
        if kernel_name and "_ZN" not in kernel_name and not _is_library_name(kernel_name):
            # a CK instance row: the reference sends every non-ASM name to the
            # CK entry, which takes no bias/alpha/beta (aiter/ops/gemm_op_a4w4.py:207-221)
            gemm_a4w4_blockscale(A.view(m, k // 2), B, A_scale, B_scale, out, splitK=split_k,
                                 kernelName=kernel_name)
            return
        gemm_a4w4_asm(A.view(m, k // 2), B, A_scale, B_scale, out, kernel_name, bias, alpha, beta,
                      bpreshuffle, log2_k_split=split_k)
    except RuntimeError as e:
        if not kernel_name or "unknown kernel name" not in str(e):
            raise
        _warn_unresolved(kernel_name, m, n, k)
        gemm_a4w4_asm(A.view(m, k // 2), B, A_scale, B_scale, out, "", bias, alpha, beta, bpreshuffle,
                      log2_k_split=0)


# names read from a tuned CSV that name no kernel of this library or of the
# reference: warned about once, then served by the heuristic
_UNRESOLVED_NAMES: set = set()


def _warn_unresolved(name: str, m: int, n: int, k: int) -> None:
    if name not in _UNRESOLVED_NAMES:
        _UNRESOLVED_NAMES.add(name)
        logger.warning(f"tuned kernel '{name}' (shape M:{m} N:{n} K:{k}) is not a kernel of this library or a "
                       f"reference tile name; using the heuristic choice")


def _is_library_name(name: str) -> bool:
    from ._lib import kernel_names

    return name in kernel_names()


def gemm_a4w4_asm(A: Tensor, B: Tensor, A_scale: Tensor, B_scale: Tensor, out: Tensor,
                  kernelName: str = "", bias: Tensor | None = None, alpha: float | None = 1.0,
                  beta: float | None = 0.0, bpreshuffle: bool | None = True,
                  log2_k_split: int | None = None) -> Tensor:
    """ctypes entry (aiter/ops/gemm_op_a4w4.py:241-287 ->
    csrc/py_itfs_cu/asm_gemm_a4w4.cu:158-278).  ``kernelName`` is one of this
    library's kernel names, or a reference ASM name
    (``_ZN5aiter..._<tM>x<tN>E``): the same tile here when this library has it
    and M > 32, else the heuristic choice; empty selects the heuristic; any
    other name raises.  D = alpha * A B^T + beta * bias."""
    call("gemm_a4w4_asm", A, B, A_scale, B_scale, out, kernelName if kernelName else None, bias,
         float(alpha if alpha is not None else 1.0), float(beta if beta is not None else 0.0),
         int(bpreshuffle) if bpreshuffle is not None else 1,
         int(log2_k_split) if log2_k_split is not None else 0)
    return out


def gemm_a4w4_blockscale(XQ: Tensor, WQ: Tensor, x_scale: Tensor, w_scale: Tensor, Out: Tensor,
                         splitK: int = 0, kernelName: str = "") -> Tensor:
    """CK-instance entry (csrc/ck_gemm_a4w4_blockscale/gemm_a4w4_blockscale.cu:69-93).
    ``splitK`` is log2 of the K split (KBatch = 2^splitK).  A kernel name of
    this library selects that instance; a CK instance name
    (``a4w4_blockscale_<block>x<tM>x<tN>x<tK>_...``) the tile of the same
    block shape here, or the heuristic choice when this library has no such
    tile; an empty name the heuristic.  Other names raise, as in the
    reference."""
    from ._lib import kernel_table

    kid = -1
    if kernelName:
        for row in kernel_table():
            if row[1] == kernelName:
                kid = row[0]
        if kid < 0:
            # resolved by name in the library (B preshuffled, no bias)
            call("gemm_a4w4_asm", XQ, WQ, x_scale, w_scale, Out, kernelName, None, 1.0, 0.0, 1,
                 int(splitK) if splitK else 0)
            return Out
    call("gemm_a4w4_blockscale", XQ, WQ, x_scale, w_scale, Out, int(splitK), int(kid))
    return Out


def gemm_a4w4_blockscale_tune(XQ: Tensor, WQ: Tensor, x_scale: Tensor, w_scale: Tensor, Out: Tensor,
                              kernelId: int = 0, splitK: int = 0) -> Tensor:
    """Tuning entry with an explicit kernel id
    (csrc/ck_gemm_a4w4_blockscale/gemm_a4w4_blockscale_tune.cu:58-90)."""
    call("gemm_a4w4_blockscale", XQ, WQ, x_scale, w_scale, Out, int(splitK), int(kernelId))
    return Out


# ---------------------------------------------------------------- low-precision outputs
# (aiter/ops/gemm_op_a4w4.py:290-409,457-567: gfx1250-only in the reference;
# here on gfx950 as the f32-output GEMM followed by one output-quant kernel)
MXFP8_OUT_SCALE_BLOCK = 128


def _is_mxfp8_out(dtype: torch.dtype) -> bool:
    return dtype == dtypes.fp8


def _alloc_f4gemm_out(M: int, N: int, dtype: torch.dtype, device) -> Tensor:
    """fp4x2 [M, N/2] (packed e2m1), fp8 [M, N] or bf16 [M, N]."""
    if dtype == dtypes.fp4x2:
        assert N % 2 == 0, "packed fp4 output requires even N"
        return torch.empty((M, N // 2), dtype=dtypes.fp4x2, device=device)
    return torch.empty((M, N), dtype=dtype, device=device)


def _alloc_f4gemm_out_scale(M: int, N: int, dtype: torch.dtype, device) -> Tensor | None:
    """MXFP8 output scale: M * N/128 e8m0 bytes in the packed (M/64, N/128, 16, 4) layout."""
    if not _is_mxfp8_out(dtype):
        return None
    assert N % MXFP8_OUT_SCALE_BLOCK == 0, f"mxfp8 output requires N % {MXFP8_OUT_SCALE_BLOCK} == 0, got N={N}"
    assert M % 64 == 0, f"mxfp8 output-scale packing requires M % 64 == 0, got M={M}"
    return torch.empty((M, N // MXFP8_OUT_SCALE_BLOCK), dtype=dtypes.fp8_e8m0, device=device)


def unpack_mxfp8_out_scale(packed: Tensor, M: int, N: int) -> Tensor:
    """Packed (M/64, N/128, 16, 4) -> row-major [M, N/128] (aiter/ops/gemm_op_a4w4.py:365-380)."""
    assert M % 64 == 0 and N % MXFP8_OUT_SCALE_BLOCK == 0
    scale_n = N // MXFP8_OUT_SCALE_BLOCK
    u8 = packed.reshape(-1).view(torch.uint8)[: (M // 64) * scale_n * 16 * 4]
    rm = u8.reshape(M // 64, scale_n, 16, 4).permute(0, 3, 2, 1).reshape(M, scale_n)
    return rm.contiguous().view(dtypes.fp8_e8m0)


def _mxfp4_gemm_asm(A: Tensor, B: Tensor, ScaleA: Tensor, ScaleB: Tensor, out: Tensor,
                    out_scale: Tensor | None = None, kernelName: str | None = None, a_preshuffle: int = 1) -> None:
    """C entry mxfp4_gemm_asm (aiter/ops/gemm_op_a4w4.py:290-304)."""
    o = out if out.dtype in (dtypes.bf16, dtypes.fp8) else out.view(torch.uint8)
    call("mxfp4_gemm_asm", A.view(torch.uint8), B.view(torch.uint8), ScaleA.view(torch.uint8),
         ScaleB.view(torch.uint8), o, None if out_scale is None else out_scale.view(torch.uint8),
         kernelName or None, int(a_preshuffle))


def gemm_mxfp4_asm(A: Tensor, B: Tensor, ScaleA: Tensor, ScaleB: Tensor, dtype: torch.dtype = dtypes.bf16,
                   a_preshuffle: bool = True, kernelName: str = ""):
    """MXFP4 GEMM with bf16 ``[M, N]``, packed-fp4 ``[M, N/2]`` (e2m1, conversion
    scale 1, input scales ignored as by the reference's packed-fp4 kernel) or
    MXFP8 ``(fp8 [M, N], packed e8m0)`` output.  A is row-major on gfx950
    (``a_preshuffle=True``, the reference's gfx1250 default, raises)."""
    M, N = A.shape[0], B.shape[0]
    out = _alloc_f4gemm_out(M, N, dtype, A.device)
    out_scale = _alloc_f4gemm_out_scale(M, N, dtype, A.device)
    _mxfp4_gemm_asm(A, B, ScaleA, ScaleB, out, out_scale, kernelName or None, int(bool(a_preshuffle)))
    return (out, out_scale) if out_scale is not None else out


def _lowp_dispatch(A, B, A_scale, B_scale, dtype, bias, alpha, beta, apreshuffle, global_A_scale, global_B_scale):
    if bias is not None or (alpha is not None and alpha != 1.0) or (beta is not None and beta != 0.0):
        logger.warning("gemm_a4w4o4/o8 ignore bias/alpha/beta (as the reference's F4GEMM kernels do)")
    if global_A_scale is not None or global_B_scale is not None:
        raise NotImplementedError("NVFP4 (per-tensor global scales) is not part of this library")
    m = A.numel() // A.shape[-1]
    return gemm_mxfp4_asm(A.view(m, A.shape[-1]), B, A_scale, B_scale, dtype=dtype,
                          a_preshuffle=bool(apreshuffle))


def gemm_a4w4o4(A: Tensor, B: Tensor, A_scale: Tensor, B_scale: Tensor, bias: Tensor | None = None,
                alpha: float | None = 1.0, beta: float | None = 0.0, bpreshuffle: bool | None = True,
                apreshuffle: bool | None = False, global_A_scale: Tensor | None = None,
                global_B_scale: Tensor | None = None) -> Tensor:
    """A4W4 GEMM with packed FP4 (e2m1, conversion scale 1) output ``[*lead, N//2]``
    (aiter/ops/gemm_op_a4w4.py:477-501)."""
    out = _lowp_dispatch(A, B, A_scale, B_scale, dtypes.fp4x2, bias, alpha, beta, apreshuffle, global_A_scale,
                         global_B_scale)
    return out.view(*A.shape[:-1], out.shape[-1])


def gemm_a4w4o8(A: Tensor, B: Tensor, A_scale: Tensor, B_scale: Tensor, bias: Tensor | None = None,
                alpha: float | None = 1.0, beta: float | None = 0.0, bpreshuffle: bool | None = True,
                apreshuffle: bool | None = False, global_A_scale: Tensor | None = None,
                global_B_scale: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """A4W4 GEMM with MXFP8 output: ``(fp8 e4m3 [*lead, N], e8m0 scale)``, the
    scale in the packed (M/64, N/128, 16, 4) layout (``unpack_mxfp8_out_scale``)
    (aiter/ops/gemm_op_a4w4.py:533-567)."""
    o, s = _lowp_dispatch(A, B, A_scale, B_scale, dtypes.fp8, bias, alpha, beta, apreshuffle, global_A_scale,
                          global_B_scale)
    lead = A.shape[:-1]
    return o.view(*lead, o.shape[-1]), s.view(*lead, s.shape[-1])
