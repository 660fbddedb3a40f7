"""CPU torch restatement of the reference's A4W4 check path.  TEST
INFRASTRUCTURE ONLY.

Only ``tests/`` and ``bench.py``'s CPU-baseline leg may import this module,
and only as the checker / the timed CPU baseline; the product path
(``aiter_amd``) never calls into it.

``run_torch_a4w4`` is ``run_torch`` of op_tests/test_gemm_a4w4.py:23-39:
unpack the e2m1 nibbles through the value table (aiter/utility/fp4_utils.py:25-52),
decode the e8m0 scales (fp4_utils.py:213-221; 0x00 -> 2^-127, 0xFF -> NaN),
repeat each scale over its 32 elements, multiply, one f32 ``torch.mm`` and a
cast to bf16.  It is pinned against the numpy oracle in tests/test_oracle.py
(dequantised operands bit-identical to ``mx_oracle.dequant_mxfp4``; the GEMM
equal to ``mx_oracle.gemm_a4w4_ref`` within f32 reordering).
"""
from __future__ import annotations

import time

import torch

SCALE_GROUP_SIZE = 32

_E2M1 = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                      -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=torch.float32)


def mxfp4_to_f32(x: torch.Tensor) -> torch.Tensor:
    """[R, K/2] packed e2m1 (uint8, even element in the low nibble) -> [R, K]
    f32 (aiter/utility/fp4_utils.py:25-52)."""
    x = x.view(torch.uint8)
    codes = torch.stack((x & 0xF, x >> 4), dim=-1).reshape(*x.shape[:-1], x.shape[-1] * 2)
    return _E2M1.to(x.device)[codes.long()]


def e8m0_to_f32(s: torch.Tensor) -> torch.Tensor:
    """e8m0 byte b -> 2^(b - 127); 0x00 -> 2^-127, 0xFF -> NaN
    (aiter/utility/fp4_utils.py:213-221)."""
    s = s.view(torch.uint8)
    bits = s.to(torch.int32) << 23
    bits = torch.where(s == 0, torch.full_like(bits, 0x00400000), bits)
    bits = torch.where(s == 0xFF, torch.full_like(bits, 0x7F800001), bits)
    return bits.view(torch.float32)


def dequant_mxfp4(x: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """[R, K/2] e2m1 + [>=R, >=K/32] plain e8m0 -> [R, K] f32."""
    v = mxfp4_to_f32(x)
    r, k = v.shape
    sc = e8m0_to_f32(scale[:r, : k // SCALE_GROUP_SIZE]).repeat_interleave(SCALE_GROUP_SIZE, dim=1)
    return v * sc


def run_torch_a4w4(x, w, x_scales, w_scales, dtype=torch.bfloat16, timings: dict | None = None):
    """op_tests/test_gemm_a4w4.py:23-39 on the CPU: dequantise A and B to f32,
    ``torch.mm(A, B^T)``, cast.  ``timings`` (if given) receives the seconds of
    the dequantisation and of the matmul separately."""
    t0 = time.perf_counter()
    a = dequant_mxfp4(x, x_scales)
    b = dequant_mxfp4(w, w_scales)
    t1 = time.perf_counter()
    c = torch.mm(a, b.T)
    t2 = time.perf_counter()
    out = c.to(dtype)
    if timings is not None:
        timings["dequant_s"] = t1 - t0
        timings["mm_s"] = t2 - t1
    return out
