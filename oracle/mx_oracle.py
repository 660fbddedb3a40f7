"""CPU oracle for the MX scaled-GEMM path.  TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import this module, and only as the checker.  The product path
(``aiter_amd``) never calls into it: a missing HIP library is an error there,
not a reason to fall back to this file.

Everything here is a numpy restatement of the reference algorithm.  Each
function cites the reference file:line it follows (paths are relative to the
aiter source tree).  Pinning status of every function (how it is checked
independently of its own formula) is listed in ``PINNED`` at the bottom and
exercised by ``tests/test_oracle.py``.

Conventions
-----------
* fp4x2: two e2m1 codes per byte, element 2i in the low nibble, 2i+1 in the
  high nibble (aiter/utility/fp4_utils.py:235-240).
* e8m0 byte b encodes 2**(b-127); 0x00 is decoded as 2**-127 and 0xFF as NaN
  (aiter/utility/fp4_utils.py:213-221).
* Round modes (csrc/include/mx_quant_utils.h:32-47):
  0 RoundDown, 1 RoundUp (default), 2 Even, 3 Ceil.
"""
from __future__ import annotations

import numpy as np

ROUND_DOWN, ROUND_UP, EVEN, CEIL = 0, 1, 2, 3

# --------------------------------------------------------------------------
# e2m1 (fp4) element codec
# --------------------------------------------------------------------------

# aiter/utility/fp4_utils.py:25-52 (mxfp4_to_f32 lookup table)
E2M1_VALUES = np.array(
    [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
     -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=np.float32)


def e2m1_decode(codes: np.ndarray) -> np.ndarray:
    """4-bit code -> float32 (aiter/utility/fp4_utils.py:25-52)."""
    return E2M1_VALUES[np.asarray(codes, dtype=np.uint8) & 0xF]


def e2m1_encode_rne(x: np.ndarray) -> np.ndarray:
    """float32 -> e2m1 code, round-to-nearest-even, saturating to +-6.

    Bit-level restatement of ``_f32_to_floatx_unpacked(x, 2, 1)``
    (aiter/utility/fp4_utils.py:255-370) and of ``fp32_to_e2m1_rne``
    (op_tests/test_quant_mxfp4.py:128-153): the saturate / denormal / normal
    branches are evaluated on the magnitude and the sign is OR-ed back in.
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.int64)
    sign = u & 0x80000000
    mag_bits = u ^ sign
    mag = mag_bits.astype(np.uint32).view(np.float32)

    saturate = mag >= 6.0
    denorm = (~saturate) & (mag < 1.0)
    normal = ~(saturate | denorm)

    # denormal branch: add 2**(149-127)... magic float so the mantissa lands
    # in the low bits (fp4_utils.py:319-327)
    denorm_const_bits = 149 << 23
    denorm_const = np.array([denorm_const_bits], dtype=np.uint32).view(np.float32)[0]
    with np.errstate(over="ignore", invalid="ignore"):
        d = (mag + denorm_const).astype(np.float32)
    d = d.view(np.uint32).astype(np.int64) - denorm_const_bits

    # normal branch: rebias the exponent and round to nearest even
    # (fp4_utils.py:329-342)
    mant_odd = (mag_bits >> 22) & 1
    val_to_add = ((1 - 127) << 23) + (1 << 21) - 1
    n = (mag_bits + val_to_add + mant_odd) >> 22

    code = np.full(u.shape, 7, dtype=np.int64)
    code = np.where(normal, n, code)
    code = np.where(denorm, d, code)
    code = code | (sign >> 28)
    return (code & 0xF).astype(np.uint8)


def pack_fp4(codes: np.ndarray) -> np.ndarray:
    """[..., 2n] codes -> [..., n] bytes, even element low (fp4_utils.py:235-240)."""
    codes = np.asarray(codes, dtype=np.uint8)
    assert codes.shape[-1] % 2 == 0
    return (codes[..., 0::2] & 0xF) | ((codes[..., 1::2] & 0xF) << 4)


def unpack_fp4(packed: np.ndarray) -> np.ndarray:
    """[..., n] bytes -> [..., 2n] codes (inverse of ``pack_fp4``)."""
    packed = np.asarray(packed, dtype=np.uint8)
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = packed & 0xF
    out[..., 1::2] = packed >> 4
    return out


def mxfp4_to_f32(packed: np.ndarray) -> np.ndarray:
    """fp4x2 bytes -> float32 values (aiter/utility/fp4_utils.py:25-52)."""
    return e2m1_decode(unpack_fp4(packed))


# --------------------------------------------------------------------------
# e4m3fn (fp8) element codec
# --------------------------------------------------------------------------

def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """OCP e4m3fn byte -> float32 (bias 7, no inf, 0x7F/0xFF = NaN)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    val = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * 2.0 ** (e - 7.0))
    val = np.where((c & 0x7F) == 0x7F, np.nan, val)
    return (s * val).astype(np.float32)


def e4m3_encode_rne(x: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn byte, round-to-nearest-even, saturating to +-448.

    The reference casts with ``.to(torch.float8_e4m3fn)``
    (op_tests/triton_tests/quant/test_quant_mxfp8.py:46) after scaling, which
    keeps |q| <= 448 by construction, so the saturation branch is unreachable
    on the quantiser path.  Restated with integer arithmetic: the magnitude is
    rounded on a grid of step 2**(e-3) (normals, e >= -6) or 2**-9 (subnormals).
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.int64)
    sign = (u >> 31) & 1
    mag_bits = u & 0x7FFFFFFF
    exp = (mag_bits >> 23) - 127          # unbiased fp32 exponent
    man = (mag_bits & 0x7FFFFF) | (1 << 23)  # 24-bit significand (normals)
    # fp32 subnormals are far below the e4m3 subnormal grid: they round to 0.
    is_f32_denorm = (mag_bits >> 23) == 0
    # quantisation step exponent: normals keep 3 mantissa bits, subnormals
    # (e < -6) sit on the fixed 2**-9 grid.
    step_e = np.maximum(exp, -6) - 3
    # significand is man * 2**(exp-23); express in units of 2**step_e
    shift = (step_e - (exp - 23)).astype(np.int64)    # >= 20
    shift = np.minimum(shift, 62)
    q = man >> shift
    rem = man - (q << shift)
    half = np.int64(1) << (shift - 1)
    round_up = (rem > half) | ((rem == half) & ((q & 1) == 1))
    q = q + round_up.astype(np.int64)
    # value = q * 2**step_e ; re-encode
    val = q.astype(np.float64) * np.exp2(step_e.astype(np.float64))
    val = np.where(is_f32_denorm, 0.0, val)
    val = np.minimum(val, 448.0)
    # encode val (exactly representable) into bits
    e_field = np.zeros_like(u)
    m_field = np.zeros_like(u)
    nz = val > 0
    with np.errstate(divide="ignore"):
        ev = np.floor(np.log2(np.where(nz, val, 1.0))).astype(np.int64)
    sub = nz & (ev < -6)
    nrm = nz & ~sub
    m_sub = np.round(np.where(sub, val, 0.0) / 2.0 ** -9).astype(np.int64)
    m_nrm = np.round((np.where(nrm, val, 1.0) / np.exp2(ev.astype(np.float64)) - 1.0) * 8).astype(np.int64)
    e_field = np.where(nrm, ev + 7, 0)
    m_field = np.where(nrm, m_nrm, np.where(sub, m_sub, 0))
    # a subnormal that rounded up to 2**-6 becomes the first normal
    carry = sub & (m_sub == 8)
    e_field = np.where(carry, 1, e_field)
    m_field = np.where(carry, 0, m_field)
    code = (sign << 7) | (e_field << 3) | m_field
    # NaN input -> 0x7F with sign (not reachable from the quantiser)
    isnan = np.isnan(x)
    code = np.where(isnan, (sign << 7) | 0x7F, code)
    return code.astype(np.uint8)


# --------------------------------------------------------------------------
# e8m0 block scales
# --------------------------------------------------------------------------

def e8m0_to_f32(b: np.ndarray) -> np.ndarray:
    """e8m0 byte -> float32 (aiter/utility/fp4_utils.py:213-221)."""
    b = np.asarray(b, dtype=np.uint8)
    bits = b.astype(np.uint32) << 23
    bits = np.where(b == 0, np.uint32(0x00400000), bits)
    bits = np.where(b == 0xFF, np.uint32(0x7F800001), bits)
    return bits.astype(np.uint32).view(np.float32)


# (target_max_pow2, inv_max_pos (f32), inv_max_pow2, even_val_to_add)
# csrc/include/mx_quant_utils.h:72-112
_FP4_CFG = (2, np.float32(1.0) / np.float32(6.0), np.float32(0.25), 0x00200000)
_FP8_CFG = (8, np.float32(1.0) / np.float32(448.0), np.float32(1.0 / 256.0), 0x00080000)


def _exp_field(f32: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(f32, dtype=np.float32).view(np.uint32) >> 23) & 0xFF


def _ceil_exp(f32: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(f32, dtype=np.float32).view(np.uint32)
    e = (bits >> 23) & 0xFF
    bump = (e < 0xFF) & ((bits & 0x7FFFFF) != 0)
    return (e + bump).astype(np.uint32)


def e8m0_scale_hip(amax: np.ndarray, mode: int, elem: str = "fp4") -> np.ndarray:
    """Per-block e8m0 byte from amax, ``fp_f32_to_e8m0_scale<mode, dtype>``
    (csrc/include/mx_quant_utils.h:130-176).

    RoundUp multiplies by the f32 constant 1/max_pos (not a division), RoundDown
    and Ceil by 1/2**target_max_pow2; Even adds ``even_val_to_add`` to the bits,
    masks the mantissa and subtracts target_max_pow2 from the exponent
    (saturating at 0).
    """
    tpow, inv_max, inv_pow2, even_add = _FP4_CFG if elem == "fp4" else _FP8_CFG
    a = np.ascontiguousarray(amax, dtype=np.float32)
    if mode == ROUND_UP:
        return _ceil_exp((a * inv_max).astype(np.float32)).astype(np.uint8)
    if mode == ROUND_DOWN:
        return _exp_field((a * inv_pow2).astype(np.float32)).astype(np.uint8)
    if mode == CEIL:
        return _ceil_exp((a * inv_pow2).astype(np.float32)).astype(np.uint8)
    if mode == EVEN:
        bits = a.view(np.uint32).astype(np.int64)
        raw = ((bits + even_add) & 0xFF800000) >> 23 & 0xFF
        return np.where(raw >= tpow, raw - tpow, 0).astype(np.uint8)
    raise ValueError(f"unknown round mode {mode}")


def e8m0_scale_log2(amax: np.ndarray, elem: str = "fp4", even_add: int = 0x200000) -> np.ndarray:
    """Even-mode scale via the floor(log2) formulation used by the Triton quant
    (aiter/utility/fp4_utils.py:413-421; fp8: ops/triton/quant test
    op_tests/triton_tests/quant/test_quant_mxfp8.py:33-41) and by
    ``quant_mxfp4_kernel`` (csrc/kernels/quant_mxfp4.cu:135-140):
    ``unbiased = clamp(floor(log2((bits(amax)+add) & 0xFF800000)) - emax, -127, 127)``,
    byte = unbiased + 127.  ``emax`` is 2 for fp4 and 8 for fp8.
    """
    emax = 2 if elem == "fp4" else 8
    a = np.ascontiguousarray(amax, dtype=np.float32)
    r = ((a.view(np.uint32).astype(np.int64) + even_add) & 0xFF800000).astype(np.uint32).view(np.float32)
    with np.errstate(divide="ignore"):
        un = np.floor(np.log2(r.astype(np.float64))) - emax
    un = np.clip(un, -127, 127)
    return (un + 127).astype(np.uint8), un


# --------------------------------------------------------------------------
# Quantisers
# --------------------------------------------------------------------------

def _groups(x: np.ndarray, group: int = 32) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    m, k = x.shape
    assert k % group == 0
    return x.reshape(m, k // group, group)


def _scaled_by_inverse(g: np.ndarray, byte: np.ndarray) -> np.ndarray:
    """x * (1/dq) with dq = 2**(byte-127) as an f32 (denormal for byte 0)."""
    dq = e8m0_to_f32_exact(byte)
    inv = np.where(dq == 0, np.float32(0), (np.float32(1) / np.where(dq == 0, 1, dq)).astype(np.float32))
    return (g * inv[..., None]).astype(np.float32)


def e8m0_to_f32_exact(b: np.ndarray) -> np.ndarray:
    """2**(b-127) as float32 including the denormal 2**-127 for b=0 (byte
    produced by ``(bits(dq) >> 23) & 0xFF`` of a pow2 f32)."""
    b = np.asarray(b, dtype=np.uint8).astype(np.float64)
    return np.exp2(b - 127).astype(np.float32)


def quant_mxfp4(x: np.ndarray, mode: int = ROUND_UP, amax_floor: float | None = None):
    """Per-1x32 MXFP4 quant -> (packed [M,K/2] u8, scale [M,K/32] u8).

    * scale byte: ``e8m0_scale_hip`` (csrc/kernels/quant_mxfp4.cu:115-148 for
      the four modes; RoundUp through csrc/kernels/quant_kernels.cu:86-120).
    * elements: RNE e2m1 of ``x * (1/2**(byte-127))``
      (op_tests/test_quant_mxfp4.py:170-179; the gfx950 hardware convert
      ``cvt_scalef32_pk_fp4`` used by both HIP kernels is byte-equal to this,
      csrc/kernels/quant_mxfp4.cu:154-167).
    * ``amax_floor``: the production RoundUp kernel starts its running max at
      1e-10f (csrc/kernels/quant_kernels.cu:89), so an all-zero block gets the
      byte of ceil_pow2(1e-10/6) instead of 0.  ``aiter_amd``'s default
      (``per_1x32_mx_quant_hip``) reproduces that; pass ``None`` for the plain
      formula used by ``quant_mxfp4_kernel`` (running max starts at 0).
    """
    g = _groups(x)
    amax = np.abs(g).max(axis=-1).astype(np.float32)
    if amax_floor is not None:
        amax = np.maximum(amax, np.float32(amax_floor))
    byte = e8m0_scale_hip(amax, mode, "fp4")
    q = e2m1_encode_rne(_scaled_by_inverse(g, byte))
    m, k = x.shape
    return pack_fp4(q.reshape(m, k)), byte


def quant_mxfp4_triton_even(x: np.ndarray):
    """Even-mode MXFP4 quant of ``dynamic_mxfp4_quant``
    (aiter/utility/fp4_utils.py:373-533, reference test restatement
    op_tests/triton_tests/quant/test_quant_mxfp4.py:18-172): scale via
    floor(log2(round(amax))) - 2, clamped to [-127,127]; elements
    RNE e2m1 of ``x * 2**-unbiased``."""
    g = _groups(x)
    amax = np.abs(g).max(axis=-1).astype(np.float32)
    byte, un = e8m0_scale_log2(amax, "fp4")
    qs = np.exp2(-un).astype(np.float32)
    q = e2m1_encode_rne((g * qs[..., None]).astype(np.float32))
    m, k = x.shape
    return pack_fp4(q.reshape(m, k)), byte


def quant_mxfp8(x: np.ndarray, mode: int = EVEN, amax_floor: float | None = None):
    """Per-1x32 MXFP8 (e4m3fn) quant -> (q [M,K] u8, scale [M,K/32] u8).

    * Even (default): Triton ``dynamic_mxfp8_quant``
      (aiter/ops/triton/_triton_kernels/quant/quant.py:380-450; restated by
      op_tests/triton_tests/quant/test_quant_mxfp8.py:24-49): amax bits
      +0x200000, floor(log2) - 8, clamp, elements ``x * 2**-unbiased`` -> e4m3.
    * RoundUp: the HIP ``per_1x32_mx_quant_hip(quant_dtype=fp8,
      scale_type=fp8_e8m0)`` path (csrc/kernels/quant_kernels.cu:86-160):
      ceil_pow2(max(amax,1e-10) * (1/448)), elements ``x * (1/scale)``.
    """
    g = _groups(x)
    amax = np.abs(g).max(axis=-1).astype(np.float32)
    if mode == EVEN:
        byte, un = e8m0_scale_log2(amax, "fp8")
        qs = np.exp2(-un).astype(np.float32)
        q = (g * qs[..., None]).astype(np.float32)
    else:
        if amax_floor is not None:
            amax = np.maximum(amax, np.float32(amax_floor))
        byte = e8m0_scale_hip(amax, mode, "fp8")
        q = _scaled_by_inverse(g, byte)
    m, k = x.shape
    return e4m3_encode_rne(q.reshape(m, k)), byte


# --------------------------------------------------------------------------
# Layouts
# --------------------------------------------------------------------------

def shuffle_weight(w: np.ndarray, layout=(16, 16)) -> np.ndarray:
    """Preshuffled-B layout (aiter/ops/shuffle.py:148-209, default branch).

    For 1-byte elements (fp4x2 / fp8 / u8) with layout (16,16): view
    (N/16, 16, Kb/32, 2, 16) and permute (0,2,3,1,4) -- i.e. per 16-row block,
    per 32-byte K chunk, per 16-byte half, the 16 rows' 16 bytes.  For 2-byte
    elements (bf16) the inner chunk is 8 elements (16 bytes).
    """
    w = np.ascontiguousarray(w)
    IN, IK = layout
    BK = IK * 2
    kpack = 16 // w.dtype.itemsize
    n, k = w.shape[-2], w.shape[-1]
    assert n % IN == 0 and k % BK == 0
    v = w.reshape(-1, n // IN, IN, k // BK, BK // kpack, kpack)
    v = v.transpose(0, 1, 3, 4, 2, 5)
    return np.ascontiguousarray(v).reshape(w.shape)


def unshuffle_weight(ws: np.ndarray, layout=(16, 16)) -> np.ndarray:
    ws = np.ascontiguousarray(ws)
    IN, IK = layout
    BK = IK * 2
    kpack = 16 // ws.dtype.itemsize
    n, k = ws.shape[-2], ws.shape[-1]
    v = ws.reshape(-1, n // IN, k // BK, BK // kpack, IN, kpack)
    v = v.transpose(0, 1, 4, 2, 3, 5)
    return np.ascontiguousarray(v).reshape(ws.shape)


def mx_scale_shuffle_idx(scale_n_pad: int, x, y):
    """Closed-form shuffled e8m0 offset of (row x, block y)
    (csrc/include/mx_quant_utils.h:212-216)."""
    x = np.asarray(x, dtype=np.int64)
    y = np.asarray(y, dtype=np.int64)
    return ((x // 32 * scale_n_pad) * 32 + (y // 8) * 256 + (y % 4) * 64
            + (x % 16) * 4 + (y % 8) // 4 * 2 + (x % 32) // 16)


def shuffle_scale(s: np.ndarray, fill: int = 0) -> np.ndarray:
    """e8m0 scale swizzle (aiter/ops/shuffle.py:339-365): pad to
    (pad256(R), pad8(C)), view (R/32, 2, 16, C/8, 2, 4), permute
    (0, 3, 5, 2, 4, 1).  Padding bytes are ``fill`` (uninitialised in the
    reference)."""
    s = np.asarray(s, dtype=np.uint8)
    m, n = s.shape
    mp, np_ = (m + 255) // 256 * 256, (n + 7) // 8 * 8
    p = np.full((mp, np_), fill, dtype=np.uint8)
    p[:m, :n] = s
    v = p.reshape(mp // 32, 2, 16, np_ // 8, 2, 4).transpose(0, 3, 5, 2, 4, 1)
    return np.ascontiguousarray(v).reshape(mp, np_)


def unshuffle_scale(ss: np.ndarray, rows: int, cols: int) -> np.ndarray:
    ss = np.asarray(ss, dtype=np.uint8)
    mp, np_ = ss.shape
    v = ss.reshape(mp // 32, np_ // 8, 4, 16, 2, 2).transpose(0, 5, 3, 1, 4, 2)
    return np.ascontiguousarray(v).reshape(mp, np_)[:rows, :cols]


def triton_scale_store_offset(scale_n_pad: int, m, n):
    """Shuffled-scale store offset of the Triton quant
    (aiter/utility/fp4_utils.py:509-525)."""
    m = np.asarray(m, dtype=np.int64)
    n = np.asarray(n, dtype=np.int64)
    o0, o1 = m // 32, m % 32
    o2, o1 = o1 % 16, o1 // 16
    o3, o4 = n // 8, n % 8
    o5, o4 = o4 % 4, o4 // 4
    return o1 + o4 * 2 + o2 * 4 + o5 * 64 + o3 * 256 + o0 * 32 * scale_n_pad


# --------------------------------------------------------------------------
# GEMM references
# --------------------------------------------------------------------------

def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit pattern, round-to-nearest-even (torch's .to(bf16))."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    return np.where(nan, np.uint16(0x7FC0), r)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def dequant_mxfp4(packed: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """[R, K/2] fp4x2 + [R, K/32] e8m0 -> [R, K] f32
    (op_tests/test_gemm_a4w4.py:28-37)."""
    v = mxfp4_to_f32(packed)
    r, k = v.shape
    s = e8m0_to_f32(np.asarray(scale)[:r, : k // 32])
    return (v.reshape(r, k // 32, 32) * s[..., None]).reshape(r, k).astype(np.float32)


def dequant_mxfp8(q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    v = e4m3_decode(q)
    r, k = v.shape
    s = e8m0_to_f32(np.asarray(scale)[:r, : k // 32])
    return (v.reshape(r, k // 32, 32) * s[..., None]).reshape(r, k).astype(np.float32)


def gemm_a4w4_ref(a_packed, b_packed, a_scale, b_scale) -> np.ndarray:
    """``run_torch`` of op_tests/test_gemm_a4w4.py:23-39: dequantise both
    operands to f32, f32 matmul A @ B^T, then bf16.  Returns bf16 bits [M,N]
    (unshuffled B / plain scales)."""
    a = dequant_mxfp4(a_packed, a_scale)
    b = dequant_mxfp4(b_packed, b_scale)
    return f32_to_bf16_bits(a @ b.T)


def gemm_a4w4_f32(a_packed, b_packed, a_scale, b_scale) -> np.ndarray:
    """The f32 product of ``gemm_a4w4_ref`` before its bf16 rounding (plain scales)."""
    return dequant_mxfp4(a_packed, a_scale) @ dequant_mxfp4(b_packed, b_scale).T


def mul_add_ref(c, a, b, fuse_type: int) -> np.ndarray:
    """Epilogue of fused_gemm_afp4wfp4_mul_add
    (aiter/ops/triton/_triton_kernels/gemm/fused/fused_gemm_afp4wfp4_mul_add.py:190-219):
    with the f32 product ``c``, ``a * c + b`` (fuse_type 0) or ``a * b + c``
    (fuse_type 1) in f32, then bf16 bits.  ``a``/``b``: numbers or arrays that
    broadcast to ``c``."""
    c = np.asarray(c, dtype=np.float32)
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32)
    out = a * c + b if fuse_type == 0 else a * b + c
    return f32_to_bf16_bits(out.astype(np.float32))


def split_cat_ref(c, y, s1: int, s2: int):
    """fused_gemm_afp4wfp4_split_cat (aiter/ops/triton/gemm/fused/fused_gemm_afp4wfp4_split_cat.py:35-39):
    ``c`` [M, D*(S1+S2)] viewed [M, D, S1+S2] is split into [..., :S1] and
    [..., S1:], and ``y`` [M, D, S3] is concatenated to the first part.
    Returns (c1 [M, D, S1+S3], c2 [M, D, S2]) of the dtype of ``c``."""
    c = np.asarray(c)
    y = np.asarray(y)
    m, d = y.shape[0], y.shape[1]
    v = c.reshape(m, d, s1 + s2)
    return np.concatenate([v[:, :, :s1], y.astype(c.dtype)], axis=2), np.ascontiguousarray(v[:, :, s1:])


def gemm_a8w4_ref(a_q, b_packed, a_scale, b_scale) -> np.ndarray:
    """MXFP8 x MXFP4: same structure with an e4m3 A (no gfx950 reference
    kernel exists; semantics from the MX spec and the gfx1250 API
    aiter/ops/gemm_op_a8w4.py:34-61)."""
    a = dequant_mxfp8(a_q, a_scale)
    b = dequant_mxfp4(b_packed, b_scale)
    return f32_to_bf16_bits(a @ b.T)


def gemm_a16w16_ref(a_bits, b_bits, bias=None) -> np.ndarray:
    """bf16 GEMM reference (op_tests/test_opus_a16w16_gemm.py:29-34):
    f32 matmul of the bf16 operands, optional f32 bias, then bf16."""
    a = bf16_bits_to_f32(a_bits)
    b = bf16_bits_to_f32(b_bits)
    c = a @ b.T
    if bias is not None:
        c = c + np.asarray(bias, dtype=np.float32)
    return f32_to_bf16_bits(c)


# --------------------------------------------------------------------------
# Dispatch helpers
# --------------------------------------------------------------------------

def get_padded_m(m: int, n: int, k: int, gl: int) -> int:
    """``getPaddedM`` (csrc/py_itfs_cu/gemm_common.cu:12-41)."""
    if gl == 0:
        if m <= 256:
            return (m + 15) // 16 * 16
        if m <= 1024:
            return (m + 31) // 32 * 32
        if m <= 4096:
            return (m + 63) // 64 * 64
        return (m + 127) // 128 * 128
    if gl == 1:
        if m > 8192 and n > 4096:
            return 8192
        return 1 if m <= 1 else 1 << (m - 1).bit_length()
    return m


# --------------------------------------------------------------------------
# Fused RMSNorm -> MX quant prologue
# --------------------------------------------------------------------------

def rms_norm_f32(x: np.ndarray, w: np.ndarray, eps: float, res: np.ndarray | None = None):
    """RMSNorm in f32 as the fused Triton kernels compute it
    (aiter/ops/triton/_triton_kernels/quant/fused_mxfp4_quant.py:8-17 and
    :119-147; fused_mxfp8_quant.py, _fused_rms_mxfp8_kernel): optional
    residual added in f32 first, then ``row * rsqrt(mean(row**2) + eps) *
    weight`` (multiplied in that order).  Returns (normed f32, x + res f32).
    The sum of squares is an f32 reduction whose order the reference leaves
    to Triton; here it is numpy's pairwise sum, so results agree with any
    other order to f32 rounding only."""
    xf = np.asarray(x, dtype=np.float32)
    if res is not None:
        xf = (xf + np.asarray(res, dtype=np.float32)).astype(np.float32)
    ss = np.sum(xf * xf, axis=-1, dtype=np.float32)
    nf = (np.float32(1.0) / np.sqrt(ss / np.float32(xf.shape[-1]) + np.float32(eps))).astype(np.float32)
    y = (xf * nf[..., None]).astype(np.float32) * np.asarray(w, dtype=np.float32)
    return y.astype(np.float32), xf


def fused_rms_mx_quant_ref(x, w, eps, fp8: bool, res=None):
    """fused_rms_mxfp4_quant / fused_rms_mxfp8_quant on one input
    (aiter/ops/triton/quant/fused_mxfp4_quant.py:23-147,
    aiter/ops/triton/quant/fused_mxfp8_quant.py:22-76): RMSNorm in f32, then
    the Even-scale quant of the f32 result (the Triton _mxfp4_quant_op /
    _mxfp8_quant_op, aiter/ops/triton/_triton_kernels/quant/quant.py:86-160,
    380-397).  Returns (q, scale [M, K/32], normed f32, x + res f32)."""
    y, xr = rms_norm_f32(x, w, eps, res)
    q, s = quant_mxfp8(y, EVEN) if fp8 else quant_mxfp4_triton_even(y)
    return q, s, y, xr


# How each function above is pinned (checked by tests/test_oracle.py).
# --------------------------------------------------------------------------
# Low-precision GEMM outputs (gemm_a4w4o4 / gemm_a4w4o8)
# --------------------------------------------------------------------------

MXFP8_OUT_BLOCK = 128


def gemm_a4w4o4_ref(a_packed, b_packed) -> np.ndarray:
    """Packed e2m1 output with conversion scale 1 and the input scales ignored
    (the reference's packed-fp4 kernel is scale-free: run_torch_mxfp4(noscale=True)
    then fp4_utils.f32_to_mxfp4, op_tests/test_f4gemm.py:108-116,224-225)."""
    c = mxfp4_to_f32(a_packed).astype(np.float64) @ mxfp4_to_f32(b_packed).astype(np.float64).T
    return pack_fp4(e2m1_encode_rne(c.astype(np.float32)))


def quant_mxfp8_block_n(x: np.ndarray, block: int = MXFP8_OUT_BLOCK):
    """``_quant_mxfp8_blockN`` of op_tests/test_f4gemm.py:70-83: per row and
    128-column block, amax (at least the smallest normal f32) -> RoundUp e8m0
    for e4m3 (ceil_pow2(amax / 448)), data = e4m3(x / scale).  Returns
    (q [M, N] u8, scale [M, N/128] u8 row-major)."""
    x = np.asarray(x, dtype=np.float32)
    m, n = x.shape
    xb = x.reshape(m, n // block, block)
    amax = np.maximum(np.abs(xb).max(axis=-1), np.float32(np.finfo(np.float32).tiny))
    byte = e8m0_scale_hip(amax, ROUND_UP, "fp8")
    q = _scaled_by_inverse(xb, byte)
    return e4m3_encode_rne(q.reshape(m, n)), byte


def pack_mxfp8_out_scale(scale_rm: np.ndarray) -> np.ndarray:
    """Row-major [M, N/128] -> the packed (M/64, N/128, 16, 4) byte layout,
    the inverse of unpack_mxfp8_out_scale (aiter/ops/gemm_op_a4w4.py:365-380):
    unpack views (M/64, N/128, 16, 4) and permutes (0, 3, 2, 1)."""
    s = np.asarray(scale_rm, dtype=np.uint8)
    m, nb = s.shape
    return np.ascontiguousarray(s.reshape(m // 64, 4, 16, nb).transpose(0, 3, 2, 1)).reshape(-1)


def unpack_mxfp8_out_scale(packed: np.ndarray, m: int, n: int) -> np.ndarray:
    """aiter/ops/gemm_op_a4w4.py:365-380."""
    nb = n // MXFP8_OUT_BLOCK
    u8 = np.asarray(packed, dtype=np.uint8).reshape(-1)[: (m // 64) * nb * 64]
    return np.ascontiguousarray(u8.reshape(m // 64, nb, 16, 4).transpose(0, 3, 2, 1)).reshape(m, nb)


def gemm_a4w4o8_ref(a_packed, b_packed, a_scale, b_scale):
    """MXFP8 output: f32 product of the dequantised operands
    (run_torch_mxfp4, op_tests/test_f4gemm.py:108-119), then quant_mxfp8_block_n.
    Returns (q [M, N] u8, scale row-major [M, N/128] u8)."""
    a = dequant_mxfp4(a_packed, a_scale)
    b = dequant_mxfp4(b_packed, b_scale)
    return quant_mxfp8_block_n((a.astype(np.float64) @ b.astype(np.float64).T).astype(np.float32))


PINNED = {
    "e2m1_decode": "OCP closed form 2**(e-1)*(1+m/2) + FP4 grid known answer",
    "e2m1_encode_rne": "brute-force nearest-grid search (ties to even code) and the "
                       "threshold form of csrc/kernels/quant_mxfp4.cu:38-55",
    "pack_fp4": "known answer {0x10,0x32,0x54,0x76} (op_tests/opus/test_opus_fp4_device.cu:88)",
    "e4m3_encode_rne": "torch .to(float8_e4m3fn) library cast + exhaustive decode round trip",
    "e8m0_scale_hip": "math.frexp / exact pow2 closed forms for each mode",
    "e8m0_scale_log2": "equal to the bit form (Even) on all test amax values",
    "quant_mxfp4": "edge values of op_tests/test_quant_mxfp4.py:352-375 + "
                   "brute-force dequant error bound; RoundUp zero-block byte pinned to the "
                   "production running-max floor only by reading (parity unpinned by test)",
    "quant_mxfp8": "torch float8_e4m3fn cast of the scaled values",
    "shuffle_weight": "explicit per-element index formula + MFMA fragment property + inverse",
    "shuffle_scale": "three formulations agree: permute, mx_scale_shuffle_idx, Triton store",
    "gemm_*_ref": "float64 brute force on tiny shapes",
    "get_padded_m": "tuned CSV keys (aiter/configs/a4w4_blockscale_tuned_gemm.csv)",
    "rms_norm_f32": "torch.nn.functional.rms_norm (library routine) in f32, and an exact case "
                    "(constant-magnitude power-of-two rows, eps 0: the factor is an exact power of two)",
    "fused_rms_mx_quant_ref": "composition of rms_norm_f32 and the pinned Even quants; exact case "
                              "bit-equal to quantising +-weight directly",
    "gemm_a4w4o4_ref": "integer brute force: fp4 codes times 4 are integers, so the product is exact and "
                       "its e2m1 code follows from the pinned encoder; float64 product",
    "quant_mxfp8_block_n": "composition of the pinned e8m0_scale_hip(RoundUp, fp8) and e4m3_encode_rne; "
                           "|q| <= 448 and dequant error <= half an e4m3 step per element",
    "pack/unpack_mxfp8_out_scale": "hand-worked known answer of the packed index and mutual inverses",
    "gemm_a4w4o8_ref": "composition of gemm_a4w4_ref's f32 product and quant_mxfp8_block_n",
}
