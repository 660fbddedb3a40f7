"""bf16 A16W16 GEMM with tuned-CSV dispatch (aiter/tuned_gemm.py:183-418, 672-727).

``gemm_a16w16(A, B, bias, otype)`` computes ``A @ B.T (+ bias)``.  The CSV row
keyed (gfx, cu_num, padded M, N, K, bias, dtype, outdtype, scaleAB,
bpreshuffle) names a backend ``libtype`` and solution (the reference's
``solMap``, aiter/tuned_gemm.py:672-680):

* ``aiter_amd``: ``solidx`` = kernel id of libaiter_amd.so (this library's
  tuner writes these rows);
* ``asm``: a reference ASM ``kernelName`` (``..._tn_<tM>x<tN>...E``) and
  ``splitK``: the same tile here when there is one, else the heuristic;
* ``opus``: ``solidx`` = a reference opus kernel id, decoded to its tile the
  same way (csrc/opus_gemm/opus_gemm_common.py:238-513);
* ``torch`` / ``hipblaslt`` / ``skinny`` / ``triton`` / ``flydsl``: backends
  that are not part of this library; the heuristic choice serves them.

Scaled bf16 (scale_a / scale_b) is out of scope and rejected.
"""
from __future__ import annotations

import functools
import os

import torch
from torch import Tensor

from . import dtypes
from ._lib import call
from .config import BF16_KEYS, DEFAULT_BF16_CSV, get_cu_num, get_gfx, load_tuned
from .gemm_common import get_padded_m

AITER_TUNE_GEMM = int(os.environ.get("AITER_TUNE_GEMM", "0"))
_UNTUNED_LOG = os.environ.get("AITER_AMD_UNTUNED_BF16_CSV", "")


@functools.lru_cache(maxsize=1)
def _bf16_table():
    return load_tuned("AITER_CONFIG_GEMM_BF16", DEFAULT_BF16_CSV, BF16_KEYS)


def _default_config():
    return {"libtype": "aiter_amd", "solidx": -1, "splitK": 0, "kernelName": ""}


@functools.lru_cache(maxsize=4096)
def get_GEMM_A16W16_config(M: int, N: int, K: int, bias: bool, dtype: str, otype: str,
                           scaleAB: bool = False, bpreshuffle: bool = False):
    """CSV lookup with the padded-M retries of aiter/tuned_gemm.py:207-300."""
    table = _bf16_table()
    gfx, cu = get_gfx(), get_cu_num()
    for gl in (None, 0, 1):
        pm = M if gl is None else get_padded_m(M, N, K, gl)
        cfg = table.get((gfx, cu, pm, N, K, bias, dtype, otype, scaleAB, bpreshuffle))
        if cfg is not None:
            return cfg
    return _default_config()


def _run(inp: Tensor, B: Tensor, bias: Tensor | None, otype: torch.dtype, bpreshuffle: bool, config,
         out: Tensor | None = None) -> Tensor:
    """Dispatch one tuned (or default) row; ``out`` may be given (the tests pass
    a NaN-filled one to see that every output tile is written)."""
    m, n = inp.shape[0], B.shape[0]
    if out is None:
        out = torch.empty((m, n), dtype=otype if otype == torch.float32 else dtypes.bf16, device=inp.device)
    libtype = config.get("libtype")
    if bias is not None and bias.dtype != torch.float32:
        bias = bias.float()
    split = int(config.get("splitK", 0) or 0)
    if libtype == "opus" and not bpreshuffle:
        call("opus_gemm_a16w16_tune", inp.unsqueeze(0), B.unsqueeze(0), out.unsqueeze(0), bias,
             int(config.get("solidx", -1)), split)
        return out
    if libtype == "aiter_amd" and int(config.get("solidx", -1)) >= 0:
        name = str(config.get("kernelName", ""))
    elif libtype == "asm":
        name = str(config.get("kernelName", "") or "")
    else:
        name, split = "", 0
    call("gemm_a16w16_asm", inp, B, out, torch.empty(0, dtype=torch.uint32, device=inp.device), bias,
         split, name or None, int(bpreshuffle))
    return out


def save_shapes(m, n, k, bias, dtype, otype, scaleAB, bpreshuffle):
    """Append untuned shapes for the tuner (aiter/tuned_gemm.py:303-333)."""
    if not AITER_TUNE_GEMM or not _UNTUNED_LOG:
        return
    new = not os.path.exists(_UNTUNED_LOG)
    with open(_UNTUNED_LOG, "a") as f:
        if new:
            f.write("M,N,K,bias,dtype,outdtype,scaleAB,bpreshuffle\n")
        f.write(f"{m},{n},{k},{bias is not None},{dtype},{otype},{scaleAB},{bpreshuffle}\n")


def gemm_a16w16(A: Tensor, B: Tensor, bias: Tensor | None = None, otype: torch.dtype | None = None,
                scale_a: Tensor | None = None, scale_b: Tensor | None = None,
                scale_c: Tensor | None = None) -> Tensor:
    if scale_a is not None or scale_b is not None or scale_c is not None:
        raise NotImplementedError("scaled bf16 GEMM is not part of this library")
    if A.dtype != dtypes.bf16 or B.dtype != dtypes.bf16:
        raise NotImplementedError("gemm_a16w16 implements bf16 inputs")
    bpreshuffle = bool(getattr(B, "is_shuffled", False))
    if A.dim() >= 3:
        inp = A.reshape(-1, A.size(-1))
        batched = True
    else:
        inp = A
        batched = False
    if not inp.is_contiguous() and inp.stride(-1) != 1:
        inp = inp.contiguous()
    m, k = inp.shape
    n = B.shape[0]
    otype = otype if otype is not None else inp.dtype
    config = get_GEMM_A16W16_config(m, n, k, bias is not None, str(inp.dtype), str(otype), False, bpreshuffle)
    out = _run(inp, B, bias, otype, bpreshuffle, config)
    if batched:
        out = out.view(*A.shape[:-1], n)
    if out.dtype != otype:
        out = out.to(otype)
    save_shapes(m, n, k, bias, inp.dtype, otype, False, bpreshuffle)
    return out


class TunedGemm:
    """``tgemm.mm`` entry (aiter/tuned_gemm.py:683-727)."""

    def mm(self, inp: Tensor, weights: Tensor, bias: Tensor | None = None, otype: torch.dtype | None = None,
           scale_a: Tensor | None = None, scale_b: Tensor | None = None, scale_c: Tensor | None = None):
        return gemm_a16w16(inp, weights, bias=bias, otype=otype, scale_a=scale_a, scale_b=scale_b,
                           scale_c=scale_c)


tgemm = TunedGemm()
