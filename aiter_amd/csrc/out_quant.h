// Low-precision GEMM outputs (aiter's gemm_a4w4o4 / gemm_a4w4o8,
// aiter/ops/gemm_op_a4w4.py:326-380,477-567): f32 [M, N] -> packed e2m1 with
// conversion scale 1 ([M, N/2]), or -> MXFP8: e4m3 [M, N] with one e8m0 scale
// per 128 columns of a row (RoundUp: ceil_pow2(amax / 448), amax at least the
// smallest normal f32), stored in the packed (M/64, N/128, 16, 4) layout
// (unpack_mxfp8_out_scale, aiter/ops/gemm_op_a4w4.py:365-380): byte (row r,
// block b) at ((r/64 * N/128 + b) * 16 + r%16) * 4 + (r%64)/16.
//
// One thread per 8 consecutive values of a row; for MXFP8 the 16 threads of a
// 128-column block (aligned lanes of one wave) reduce amax with shuffles.
// Conversions are gfx950's scaled pair instructions (RNE, saturating), the
// bytes of the software conversions for every finite input.
#pragma once
#include "mx_quant.h"

namespace aiter_amd {

template <bool FP8>
__global__ __launch_bounds__(256) void out_quant_kernel(const float* in, int64_t M, int64_t N, int64_t in_stride,
                                                        uint8_t* out, int64_t out_stride, uint8_t* scale) {
    using namespace mx;
    const int64_t per_row = N / 8;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const bool live = gid < M * per_row;
    const int64_t row = live ? gid / per_row : 0;
    const int64_t c8 = live ? gid % per_row : 0;
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (live) {
        const f32x4_t a = *reinterpret_cast<const f32x4_t*>(in + row * in_stride + c8 * 8);
        const f32x4_t b = *reinterpret_cast<const f32x4_t*>(in + row * in_stride + c8 * 8 + 4);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            v[k] = a[k];
            v[4 + k] = b[k];
        }
    }
    if constexpr (!FP8) {
        if (!live) return;
        uint32_t w = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) w = cvt_fp4_pair<float>(w, 0u, v[2 * j], v[2 * j + 1], 1.0f, j);
        *reinterpret_cast<uint32_t*>(out + row * out_stride + c8 * 4) = w;
    } else {
        float amax = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[k]));
#pragma unroll
        for (int d = 1; d < 16; d <<= 1) amax = __builtin_fmaxf(amax, __shfl_xor(amax, d));
        if (!live) return;
        amax = __builtin_fmaxf(amax, 1.17549435e-38f);
        const uint32_t byte = e8m0_byte<kRoundUp>(amax, 1.0f / 448.0f, 1.0f / 256.0f, 0u, 8u);
        uint32_t w0 = 0, w1 = 0;
        if (byte != 0u && byte != 255u) {
            const float ds = __builtin_bit_cast(float, byte << 23);
            w0 = cvt_fp8_pair<float>(w0, 0u, v[0], v[1], ds, false);
            w0 = cvt_fp8_pair<float>(w0, 0u, v[2], v[3], ds, true);
            w1 = cvt_fp8_pair<float>(w1, 0u, v[4], v[5], ds, false);
            w1 = cvt_fp8_pair<float>(w1, 0u, v[6], v[7], ds, true);
        } else {
            const float inv = inv_scale_from_byte(byte);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                w0 |= f32_to_e4m3(v[k] * inv) << (8 * k);
                w1 |= f32_to_e4m3(v[4 + k] * inv) << (8 * k);
            }
        }
        *reinterpret_cast<uint2*>(out + row * out_stride + c8 * 8) = uint2{w0, w1};
        if ((c8 & 15) == 0) {
            const int64_t nb = N / 128, b = c8 / 16;
            scale[((row / 64 * nb + b) * 16 + row % 16) * 4 + (row % 64) / 16] = (uint8_t)byte;
        }
    }
}

}  // namespace aiter_amd
