// Per-1x32 MX block helpers shared by the quantisers (quant.hip) and the
// fused RMSNorm -> MX quant prologue (fused_quant.hip): e8m0 scale bytes for
// the four rounding modes, the scaled pair conversions of gfx950 and their
// integer equivalents, and the shuffled-scale index.
#pragma once
#include <type_traits>

#include "common.h"

namespace aiter_amd {
namespace mx {

enum ScaleMode : int { kRoundDown = 0, kRoundUp = 1, kEven = 2, kCeil = 3 };

// e8m0 byte of a block, following fp_f32_to_e8m0_scale<mode, dtype>
// (csrc/include/mx_quant_utils.h:130-176).  `even_add`/`emax` give the Even
// rounding constants (0x200000/2 for fp4, 0x200000/8 for the Triton MXFP8
// quant of aiter/ops/triton/_triton_kernels/quant/quant.py).
template <int MODE>
AA_DEV uint32_t e8m0_byte(float amax, float inv_max_pos, float inv_max_pow2, uint32_t even_add,
                          uint32_t emax) {
    if constexpr (MODE == kRoundUp || MODE == kCeil) {
        const float t = (MODE == kRoundUp) ? amax * inv_max_pos : amax * inv_max_pow2;
        const uint32_t u = __builtin_bit_cast(uint32_t, t);
        uint32_t e = (u >> 23) & 0xffu;
        if (e < 0xffu && (u & 0x7fffffu)) e += 1;
        return e;
    } else if constexpr (MODE == kRoundDown) {
        return (__builtin_bit_cast(uint32_t, amax * inv_max_pow2) >> 23) & 0xffu;
    } else {
        const uint32_t r = ((__builtin_bit_cast(uint32_t, amax) + even_add) & 0xff800000u) >> 23 & 0xffu;
        return r >= emax ? r - emax : 0u;
    }
}

// 2^(127-byte) as f32 (the quantisation multiplier 1/scale; 2^-127 is the
// f32 subnormal 0x00400000).
AA_DEV float inv_scale_from_byte(uint32_t b) {
    if (b == 254u) return __builtin_bit_cast(float, 0x00400000u);
    return __builtin_bit_cast(float, (254u - b) << 23);
}

// f32 -> e2m1 code (RNE, saturating to 6), the bit-level algorithm of
// _f32_to_floatx_unpacked (aiter/utility/fp4_utils.py:255-370).
AA_DEV uint32_t f32_to_e2m1(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const uint32_t s = u & 0x80000000u;
    const uint32_t a = u ^ s;
    const float af = __builtin_bit_cast(float, a);
    uint32_t code;
    if (af >= 6.0f) {
        code = 7u;
    } else if (af < 1.0f) {
        const float d = af + __builtin_bit_cast(float, 149u << 23);
        code = __builtin_bit_cast(uint32_t, d) - (149u << 23);
    } else {
        const uint32_t odd = (a >> 22) & 1u;
        code = (a + ((uint32_t)(1 - 127) << 23) + (1u << 21) - 1u + odd) >> 22;
    }
    return (code | (s >> 28)) & 0xfu;
}

// f32 -> e4m3fn byte (RNE, saturating to 448, NaN -> 0x7f).
AA_DEV uint32_t f32_to_e4m3(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const uint32_t s = (u >> 24) & 0x80u;
    const uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return s | 0x7fu;
    uint32_t code;
    if (a < (121u << 23)) {  // |x| < 2^-6: subnormal grid of step 2^-9
        const float q = __builtin_rintf(__builtin_bit_cast(float, a) * 512.0f);
        code = (uint32_t)q;  // 0..8 (8 == first normal)
    } else {
        uint32_t r = (a + 0x7ffffu + ((a >> 20) & 1u)) >> 20;
        r -= 120u << 3;
        code = r > 0x7eu ? 0x7eu : r;
    }
    return s | code;
}

// One scaled pair conversion; `sel` (byte of the destination) must fold to a
// constant.  InT selects the source form: bf16 pair, f16 pair (both as the
// raw 32-bit pair) or two f32 values.
template <typename InT>
AA_DEV uint32_t cvt_fp4_pair(uint32_t old, uint32_t pair, float a, float b, float scale, int sel) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
#define AA_CVT_SEL(S)                                                                                   \
    case S:                                                                                             \
        if constexpr (std::is_same<InT, float>::value)                                                  \
            return __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(old, a, b, scale, S);                       \
        else if constexpr (std::is_same<InT, _Float16>::value)                                          \
            return __builtin_amdgcn_cvt_scalef32_pk_fp4_f16(old, __builtin_bit_cast(f16x2_t, pair), scale, S); \
        else                                                                                            \
            return __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16(old, __builtin_bit_cast(bf16x2_t, pair), scale, S);
    switch (sel) {
        AA_CVT_SEL(0) AA_CVT_SEL(1) AA_CVT_SEL(2) AA_CVT_SEL(3)
    }
#undef AA_CVT_SEL
    return old;
}

// Scaled pair conversion to e4m3fn: two values / scale -> two bytes in word
// `hi` (0 or 1, constant) of the destination.
template <typename InT>
AA_DEV uint32_t cvt_fp8_pair(uint32_t old, uint32_t pair, float a, float b, float scale, bool hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    typedef short s16x2_t __attribute__((ext_vector_type(2)));
    const s16x2_t o = __builtin_bit_cast(s16x2_t, old);
    s16x2_t r;
    if constexpr (std::is_same<InT, float>::value)
        r = hi ? __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(o, a, b, scale, true)
               : __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(o, a, b, scale, false);
    else if constexpr (std::is_same<InT, _Float16>::value)
        r = hi ? __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(o, __builtin_bit_cast(f16x2_t, pair), scale, true)
               : __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(o, __builtin_bit_cast(f16x2_t, pair), scale, false);
    else
        r = hi ? __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(o, __builtin_bit_cast(bf16x2_t, pair), scale, true)
               : __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(o, __builtin_bit_cast(bf16x2_t, pair), scale, false);
    return __builtin_bit_cast(uint32_t, r);
}

// e2m1 codes of one 32-element block held in registers: v = the 32 values
// as f32, raw = the 16 element pairs as loaded (16-bit InT; unused for f32).
// Returns the e8m0 byte (MODE, with the running max starting at amax_floor)
// and the 16 code bytes in o (even element in the low nibble).  Bytes 1..254
// take gfx950's scaled pair conversion (value / 2^(byte-127), RNE,
// saturating), 0 and 255 the integer conversion of value * 2^(127-byte):
// the same codes either way.
template <typename InT, int MODE>
AA_DEV uint32_t quant32_fp4(const float (&v)[32], const uint32_t (&raw)[16], float amax_floor, float inv_max_pos,
                            float inv_max_pow2, uint32_t even_add, uint32_t emax, i32x4_t& o) {
    float amax = amax_floor;
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[i]));
    const uint32_t byte = e8m0_byte<MODE>(amax, inv_max_pos, inv_max_pow2, even_add, emax);
    const float inv = inv_scale_from_byte(byte);
    if (byte != 0u && byte != 255u) {
        const float ds = __builtin_bit_cast(float, byte << 23);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t w = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (sizeof(InT) == 2)
                    w = cvt_fp4_pair<InT>(w, raw[i * 4 + j], 0.f, 0.f, ds, j);
                else
                    w = cvt_fp4_pair<float>(w, 0u, v[i * 8 + 2 * j], v[i * 8 + 2 * j + 1], ds, j);
            }
            o[i] = (int)w;
        }
    } else {
        // scale byte 0 (2^-127, a subnormal f32) or 255 (NaN)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t w = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) w |= f32_to_e2m1(v[i * 8 + j] * inv) << (4 * j);
            o[i] = (int)w;
        }
    }
    return byte;
}

AA_DEV int scale_shuffle_idx(int scale_n_pad, int x, int y) {
    // csrc/include/mx_quant_utils.h:212-216
    return (x / 32 * scale_n_pad) * 32 + (y / 8) * 256 + (y % 4) * 64 + (x % 16) * 4 +
           (y % 8) / 4 * 2 + (x % 32) / 16;
}

}  // namespace mx
}  // namespace aiter_amd
