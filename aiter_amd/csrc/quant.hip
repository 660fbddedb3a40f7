// Per-1x32 MX activation/weight quantisers (MXFP4 e2m1 / MXFP8 e4m3fn with
// e8m0 block scales) for gfx950.
//
// One thread owns one 32-element block: it reads the block with 16-byte
// vector loads (consecutive threads read consecutive blocks of a row, so a
// wave covers 2-4 KiB of contiguous input), reduces amax in registers, derives
// the e8m0 byte, converts the 32 values and writes 16 B (fp4) or 32 B (fp8)
// plus one scale byte.  The work is HBM-bound: 64 B in / 17 B out per block
// for bf16 -> fp4.
//
// Element conversion: gfx950's scaled pair conversions
// (v_cvt_scalef32_pk_fp4_* / v_cvt_scalef32_pk_fp8_*: value / 2^(e-127),
// round to nearest even, saturating) for scale bytes 1..254, and integer
// arithmetic (RNE) for the two bytes whose scale is not a normal f32 (0:
// 2^-127, 255).  Both give the reference CPU restatements' bytes; the
// hardware form costs one instruction per pair instead of ~15 per element,
// which moves the kernel from VALU-bound to HBM-bound.

#include "common.h"
#include "mx_quant.h"

namespace {

using namespace aiter_amd::mx;

struct QuantParams {
    const void* in;
    uint8_t* out;
    uint8_t* scale;
    int64_t rows;          // rows to quantise
    int64_t cover_rows;    // rows whose scale bytes are written (>= rows; extra -> 0)
    int64_t in_stride;     // elements
    int64_t out_stride;    // bytes
    int64_t scale_stride;  // bytes (plain layout)
    int scale_n;           // valid blocks per row
    int scale_n_pad;       // blocks per row in the grid (>= scale_n)
    int cols;              // elements per row
    const int* num_rows;   // optional device row count
    int num_rows_factor;
    int shuffle_scale;
    int shuffle_weight;    // fused preshuffle of the packed fp4 output
    int zero_pad;          // write 0 into padding blocks of a shuffled scale buffer
    float inv_max_pos, inv_max_pow2;
    uint32_t even_add, emax;
    float amax_floor;
};

template <typename InT, bool OUT_FP8, int MODE>
__global__ __launch_bounds__(256) void mx_quant_kernel(QuantParams p) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t x = gid / p.scale_n_pad;
    const int y = (int)(gid % p.scale_n_pad);
    int64_t rows = p.rows;
    if (p.num_rows) rows = (int64_t)(*p.num_rows) * p.num_rows_factor;
    if (x >= p.cover_rows) return;
    const bool valid = (x < rows) && (y < p.scale_n);
    if (!valid) {
        // padding of the (Triton-layout) shuffled scale buffer is written as zero
        if (p.zero_pad) p.scale[scale_shuffle_idx(p.scale_n_pad, (int)x, y)] = 0;
        return;
    }

    constexpr int kVec = 16 / sizeof(InT);  // elements per 16-byte load
    float v[32];
    uint32_t raw[sizeof(InT) == 2 ? 16 : 1];   // 16-bit inputs: the loaded element pairs
    const InT* src = reinterpret_cast<const InT*>(p.in) + x * p.in_stride + (int64_t)y * 32;
#pragma unroll
    for (int i = 0; i < 32 / kVec; ++i) {
        const i32x4_t w = *reinterpret_cast<const i32x4_t*>(src + i * kVec);
        if constexpr (sizeof(InT) == 4) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                // copy the lane to a scalar first: bit-casting the vector
                // element expression directly reads element 0 (clang 22)
                const int e = w[j];
                v[i * 4 + j] = __builtin_bit_cast(float, e);
            }
        } else if constexpr (std::is_same<InT, _Float16>::value) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t d = (uint32_t)w[j];
                raw[i * 4 + j] = d;
                v[i * 8 + 2 * j] = (float)__builtin_bit_cast(_Float16, (uint16_t)(d & 0xffffu));
                v[i * 8 + 2 * j + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(d >> 16));
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t d = (uint32_t)w[j];
                raw[i * 4 + j] = d;
                v[i * 8 + 2 * j] = __builtin_bit_cast(float, d << 16);
                v[i * 8 + 2 * j + 1] = __builtin_bit_cast(float, d & 0xffff0000u);
            }
        }
    }
    float amax = p.amax_floor;
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[i]));

    const uint32_t byte = e8m0_byte<MODE>(amax, p.inv_max_pos, p.inv_max_pow2, p.even_add, p.emax);
    const float inv = inv_scale_from_byte(byte);

    if constexpr (OUT_FP8) {
        i32x4_t o[2];
        if (byte != 0u && byte != 255u) {
            const float ds = __builtin_bit_cast(float, byte << 23);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                uint32_t w = 0;
                if constexpr (sizeof(InT) == 2) {
                    w = cvt_fp8_pair<InT>(w, raw[2 * i], 0.f, 0.f, ds, false);
                    w = cvt_fp8_pair<InT>(w, raw[2 * i + 1], 0.f, 0.f, ds, true);
                } else {
                    w = cvt_fp8_pair<float>(w, 0u, v[4 * i], v[4 * i + 1], ds, false);
                    w = cvt_fp8_pair<float>(w, 0u, v[4 * i + 2], v[4 * i + 3], ds, true);
                }
                o[i / 4][i % 4] = (int)w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                uint32_t w = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) w |= f32_to_e4m3(v[i * 4 + j] * inv) << (8 * j);
                o[i / 4][i % 4] = (int)w;
            }
        }
        uint8_t* dst = p.out + x * p.out_stride + (int64_t)y * 32;
        *reinterpret_cast<i32x4_t*>(dst) = o[0];
        *reinterpret_cast<i32x4_t*>(dst + 16) = o[1];
    } else {
        i32x4_t o;
        if (byte != 0u && byte != 255u) {
            // gfx950 v_cvt_scalef32_pk_fp4_*: two values / 2^(byte-127) -> two
            // e2m1 nibbles (RNE, saturating at 6; the even element in the low
            // nibble), placed in byte `sel` of the destination: the same
            // codes as f32_to_e2m1(x * 2^(127-byte)) below for every finite
            // input, in one instruction per pair
            const float ds = __builtin_bit_cast(float, byte << 23);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t w = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if constexpr (std::is_same<InT, _Float16>::value)
                        w = cvt_fp4_pair<_Float16>(w, raw[i * 4 + j], 0.f, 0.f, ds, j);
                    else if constexpr (sizeof(InT) == 2)
                        w = cvt_fp4_pair<uint16_t>(w, raw[i * 4 + j], 0.f, 0.f, ds, j);
                    else
                        w = cvt_fp4_pair<float>(w, 0u, v[i * 8 + 2 * j], v[i * 8 + 2 * j + 1], ds, j);
                }
                o[i] = (int)w;
            }
        } else {
            // scale byte 0 (2^-127, a subnormal f32) or 255 (NaN): the
            // integer conversion
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t w = 0;
#pragma unroll
                for (int j = 0; j < 8; ++j) w |= f32_to_e2m1(v[i * 8 + j] * inv) << (4 * j);
                o[i] = (int)w;
            }
        }
        int64_t off;
        if (p.shuffle_weight) {
            // shuffle_weight((16,16)) position of bytes [16y, 16y+16) of row x
            // (aiter/ops/shuffle.py:192-204; fused form csrc/kernels/quant_mxfp4.cu:177-183)
            off = (x >> 4) * 16 * p.out_stride + (x & 15) * 16 + (int64_t)(y >> 1) * 512 + (y & 1) * 256;
        } else {
            off = x * p.out_stride + (int64_t)y * 16;
        }
        *reinterpret_cast<i32x4_t*>(p.out + off) = o;
    }
    if (p.shuffle_scale)
        p.scale[scale_shuffle_idx(p.scale_n_pad, (int)x, y)] = (uint8_t)byte;
    else
        p.scale[x * p.scale_stride + y] = (uint8_t)byte;
}

template <typename InT, bool OUT_FP8>
void launch_mode(int mode, const QuantParams& p, int64_t nthreads, hipStream_t st) {
    const dim3 grid((unsigned)((nthreads + 255) / 256));
    switch (mode) {
        case kRoundDown: mx_quant_kernel<InT, OUT_FP8, kRoundDown><<<grid, 256, 0, st>>>(p); break;
        case kRoundUp: mx_quant_kernel<InT, OUT_FP8, kRoundUp><<<grid, 256, 0, st>>>(p); break;
        case kEven: mx_quant_kernel<InT, OUT_FP8, kEven><<<grid, 256, 0, st>>>(p); break;
        case kCeil: mx_quant_kernel<InT, OUT_FP8, kCeil><<<grid, 256, 0, st>>>(p); break;
        default: aiter_amd::fail("quant", "round_mode must be 0..3, got ", mode);
    }
}

struct QuantRequest {
    const aiter_tensor_t* x;
    const aiter_tensor_t* out;
    const aiter_tensor_t* scale;
    bool out_fp8;
    int mode;
    bool shuffle_scale;
    bool shuffle_weight;
    bool zero_pad_scale;   // Triton layout: write 0 into rows M..pad32(M) and cols scaleN..pad8
    float amax_floor;
    uint32_t even_add;
    const int* num_rows;
    int num_rows_factor;
};

void run_quant(const QuantRequest& q, hipStream_t stream) {
    using namespace aiter_amd;
    check_tensor(q.x, "input");
    check_tensor(q.out, "out");
    check_tensor(q.scale, "scale");
    const int in_dt = q.x->dtype;
    AA_CHECK(in_dt == AITER_DTYPE_bf16 || in_dt == AITER_DTYPE_fp16 || in_dt == AITER_DTYPE_fp32,
             "input must be bf16/fp16/fp32, got ", dtype_name(in_dt));
    const int64_t rows = rows_2d(q.x);
    const int64_t cols = cols_2d(q.x);
    AA_CHECK(cols % 32 == 0, "last dim ", cols, " must be a multiple of 32");
    const int64_t in_stride = row_stride_2d(q.x, "input");
    AA_CHECK(in_stride % (16 / dtype_size(in_dt)) == 0, "input row stride must keep 16-byte alignment");
    AA_CHECK(((uintptr_t)q.x->ptr & 15) == 0, "input must be 16-byte aligned");
    AA_CHECK(is_byte_type(q.out->dtype), "out must be a 1-byte dtype (fp4x2/fp8/u8)");
    AA_CHECK(is_byte_type(q.scale->dtype), "scale must be e8m0/u8 (fp32 scales are not produced here)");
    AA_CHECK(rows_2d(q.out) == rows, "out rows ", rows_2d(q.out), " != input rows ", rows);
    const int64_t out_cols = q.out_fp8 ? cols : cols / 2;
    AA_CHECK(cols_2d(q.out) == out_cols, "out last dim ", cols_2d(q.out), " != ", out_cols);
    const int64_t out_stride = row_stride_2d(q.out, "out");
    AA_CHECK(out_stride % 16 == 0 && ((uintptr_t)q.out->ptr & 15) == 0,
             "out rows must be 16-byte aligned");
    if (q.shuffle_weight) {
        AA_CHECK(!q.out_fp8, "shuffle_weight is only defined for fp4 output");
        AA_CHECK(rows % 16 == 0 && out_cols % 32 == 0 && out_stride == out_cols,
                 "shuffle_weight needs rows%16==0, K/2%32==0 and a contiguous output");
    }
    const int scale_n = (int)(cols / 32);
    const int scale_n_pad = q.shuffle_scale ? (scale_n + 7) / 8 * 8 : scale_n;
    const int64_t cover_rows = (q.shuffle_scale && q.zero_pad_scale) ? (rows + 31) / 32 * 32 : rows;
    int64_t scale_stride = 0;
    if (q.shuffle_scale) {
        const int64_t need = (rows + 255) / 256 * 256 * (int64_t)scale_n_pad;
        AA_CHECK((int64_t)q.scale->numel >= need, "shuffled scale needs [pad256(M), pad8(K/32)] = ",
                 need, " bytes, got ", q.scale->numel);
        AA_CHECK(cols_2d(q.scale) == scale_n_pad || q.scale->ndim == 1,
                 "shuffled scale last dim must be pad8(K/32) = ", scale_n_pad);
    } else {
        AA_CHECK(rows_2d(q.scale) >= rows && cols_2d(q.scale) >= scale_n,
                 "scale must be at least [M, K/32] = [", rows, ", ", scale_n, "]");
        scale_stride = row_stride_2d(q.scale, "scale");
    }
    if (rows == 0) return;

    QuantParams p{};
    p.in = q.x->ptr;
    p.out = static_cast<uint8_t*>(q.out->ptr);
    p.scale = static_cast<uint8_t*>(q.scale->ptr);
    p.rows = rows;
    p.cover_rows = cover_rows;
    p.in_stride = in_stride;
    p.out_stride = out_stride;
    p.scale_stride = scale_stride;
    p.scale_n = scale_n;
    p.scale_n_pad = scale_n_pad;
    p.zero_pad = q.shuffle_scale && q.zero_pad_scale;
    p.cols = (int)cols;
    p.num_rows = q.num_rows;
    p.num_rows_factor = q.num_rows_factor;
    p.shuffle_scale = q.shuffle_scale;
    p.shuffle_weight = q.shuffle_weight;
    if (q.out_fp8) {
        p.inv_max_pos = 1.0f / 448.0f;
        p.inv_max_pow2 = 1.0f / 256.0f;
        p.emax = 8;
    } else {
        p.inv_max_pos = 1.0f / 6.0f;
        p.inv_max_pow2 = 0.25f;
        p.emax = 2;
    }
    p.even_add = q.even_add;
    p.amax_floor = q.amax_floor;
    // the grid walks scale_n_pad blocks per row so padding columns are covered
    const int64_t nthreads = cover_rows * (int64_t)p.scale_n_pad;
    AA_CHECK(nthreads / 256 < ((int64_t)1 << 31), "problem too large for one launch");

    if (in_dt == AITER_DTYPE_bf16) {
        if (q.out_fp8) launch_mode<uint16_t, true>(q.mode, p, nthreads, stream);
        else launch_mode<uint16_t, false>(q.mode, p, nthreads, stream);
    } else if (in_dt == AITER_DTYPE_fp16) {
        if (q.out_fp8) launch_mode<_Float16, true>(q.mode, p, nthreads, stream);
        else launch_mode<_Float16, false>(q.mode, p, nthreads, stream);
    } else {
        if (q.out_fp8) launch_mode<float, true>(q.mode, p, nthreads, stream);
        else launch_mode<float, false>(q.mode, p, nthreads, stream);
    }
    AA_HIP(hipGetLastError());
}

}  // namespace

extern "C" {

int dynamic_per_group_scaled_quant(aiter_tensor_t* out, aiter_tensor_t* input,
                                   aiter_tensor_t* scales, int group_size, int shuffle_scale,
                                   aiter_tensor_t* num_rows, int num_rows_factor,
                                   aiter_stream_t stream) {
    return aiter_amd::safe_call([&] {
        AA_CHECK(group_size == 32, "only group_size 32 (MX) is implemented, got ", group_size);
        aiter_amd::check_tensor(out, "out");
        aiter_amd::DeviceGuard g(input ? input->device_id : -1);
        QuantRequest q{};
        q.x = input;
        q.out = out;
        q.scale = scales;
        q.out_fp8 = out->dtype == AITER_DTYPE_fp8;
        AA_CHECK(q.out_fp8 || out->dtype == AITER_DTYPE_fp4x2 || out->dtype == AITER_DTYPE_u8,
                 "out must be fp4x2 or fp8");
        q.mode = kRoundUp;  // kDefaultMxScaleRoundMode (csrc/include/mx_quant_utils.h:49)
        q.shuffle_scale = shuffle_scale != 0;
        q.amax_floor = 1e-10f;  // running max start of csrc/kernels/quant_kernels.cu:89
        q.even_add = 0;
        q.num_rows = num_rows ? static_cast<const int*>(num_rows->ptr) : nullptr;
        q.num_rows_factor = num_rows_factor;
        run_quant(q, reinterpret_cast<hipStream_t>(stream));
    });
}

int quant_mxfp4(aiter_tensor_t* x, aiter_tensor_t* out_packed, aiter_tensor_t* out_scale,
                int group_size, int round_mode, int e8m0_shuffle, int a16w4_shuffle, int gate_up,
                int shuffle_weight, aiter_stream_t stream) {
    return aiter_amd::safe_call([&] {
        AA_CHECK(group_size == 32, "only group_size 32 is implemented, got ", group_size);
        AA_CHECK(!a16w4_shuffle && !gate_up, "a16w4/gate_up (MoE) layouts are not part of this library");
        AA_CHECK(round_mode >= 0 && round_mode <= 3, "round_mode must be 0..3, got ", round_mode);
        aiter_amd::DeviceGuard g(x ? x->device_id : -1);
        QuantRequest q{};
        q.x = x;
        q.out = out_packed;
        q.scale = out_scale;
        q.out_fp8 = false;
        q.mode = round_mode;
        q.shuffle_scale = e8m0_shuffle != 0;
        q.shuffle_weight = shuffle_weight != 0;
        q.amax_floor = 0.0f;  // csrc/kernels/quant_mxfp4.cu:108
        q.even_add = 0x200000u;
        run_quant(q, reinterpret_cast<hipStream_t>(stream));
    });
}

int dynamic_mxfp4_quant(aiter_tensor_t* x, aiter_tensor_t* x_fp4, aiter_tensor_t* scale,
                        int shuffle, aiter_stream_t stream) {
    return aiter_amd::safe_call([&] {
        aiter_amd::DeviceGuard g(x ? x->device_id : -1);
        QuantRequest q{};
        q.x = x;
        q.out = x_fp4;
        q.scale = scale;
        q.out_fp8 = false;
        q.mode = kEven;
        q.shuffle_scale = shuffle != 0;
        q.zero_pad_scale = true;
        q.amax_floor = 0.0f;
        q.even_add = 0x200000u;
        run_quant(q, reinterpret_cast<hipStream_t>(stream));
    });
}

int dynamic_mxfp8_quant(aiter_tensor_t* x, aiter_tensor_t* y, aiter_tensor_t* scale, int shuffle,
                        aiter_stream_t stream) {
    return aiter_amd::safe_call([&] {
        aiter_amd::DeviceGuard g(x ? x->device_id : -1);
        QuantRequest q{};
        q.x = x;
        q.out = y;
        q.scale = scale;
        q.out_fp8 = true;
        q.mode = kEven;
        q.shuffle_scale = shuffle != 0;
        q.zero_pad_scale = shuffle != 0;
        q.amax_floor = 0.0f;
        q.even_add = 0x200000u;  // aiter/ops/triton/_triton_kernels/quant/quant.py (0x200000, -8)
        run_quant(q, reinterpret_cast<hipStream_t>(stream));
    });
}

}  // extern "C"
