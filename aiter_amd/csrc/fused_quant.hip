// Fused RMSNorm -> MX quant prologue for gfx950: the producer of the
// activation operand of the A4W4 / A8W4 GEMMs, in one pass over HBM instead
// of a normalisation kernel followed by a quantiser.
//
// Follows fused_rms_mxfp4_quant (aiter/ops/triton/quant/fused_mxfp4_quant.py:
// 23-147; kernel aiter/ops/triton/_triton_kernels/quant/fused_mxfp4_quant.py:
// 8-222) and fused_rms_mxfp8_quant (aiter/ops/triton/quant/fused_mxfp8_quant.py:
// 22-76): optional residual x1 += res1 in f32 (stored back as out_res1),
// y = x1 * rsqrt(mean(x1^2) + eps) * weight in f32, optional unquantised y
// (out1), the Even-scale MX quant of the f32 y; optionally a second input x2
// RMS-normalised without quantisation (out2).
//
// One workgroup of 256 threads per row; thread t owns the 32-element blocks
// t, t+256, ... (up to kMaxBlocks of them, kept in registers between the
// two passes), so the row is read once.  The sum of squares is reduced per
// thread in block order, then across the workgroup (DPP within waves, LDS
// across them); 1/sqrt is v_rsq_f32.

#include "common.h"
#include "mx_quant.h"

namespace {

using namespace aiter_amd::mx;

constexpr int kThreads = 256;
constexpr int kMaxBlocks = 4;   // rows up to 4 * 256 * 32 = 32768 elements

struct RmsQuantParams {
    const void* x1;
    const void* w1;
    const void* res1;
    const void* x2;
    const void* w2;
    uint8_t* q;           // [M, N1/2] e2m1 pairs or [M, N1] e4m3
    uint8_t* scale;       // [M, N1/32] or shuffled [pad256(M), pad8(N1/32)]
    void* out1;           // optional unquantised y (x1's dtype)
    void* out2;           // optional RMSNorm(x2) (x1's dtype)
    void* out_res1;       // optional x1 + res1 (x1's dtype)
    float eps1, eps2;
    int M, N1, N2;
    int64_t x1_stride, res1_stride, x2_stride, q_stride, scale_stride, out1_stride, out2_stride, out_res1_stride;
    int shuffle;          // shuffled scale layout
    int pad_scale;        // write 127 into blocks [N1/32, pad8(N1/32)) of each row
    int scale_n_pad;
};

template <typename T>
AA_DEV float to_f32(T v) {
    if constexpr (std::is_same<T, float>::value) return v;
    else if constexpr (std::is_same<T, _Float16>::value) return (float)v;
    else return __builtin_bit_cast(float, (uint32_t)__builtin_bit_cast(uint16_t, v) << 16);
}

template <typename T>
AA_DEV T from_f32(float f) {
    if constexpr (std::is_same<T, float>::value) return f;
    else if constexpr (std::is_same<T, _Float16>::value) return (_Float16)f;
    else return __builtin_bit_cast(T, __builtin_bit_cast(uint16_t, (__bf16)f));
}

// 32 elements of a row as f32 (16-byte loads)
template <typename T>
AA_DEV void load32(const T* src, float (&v)[32]) {
    constexpr int kVec = 16 / sizeof(T);
#pragma unroll
    for (int i = 0; i < 32 / kVec; ++i) {
        const i32x4_t w = *reinterpret_cast<const i32x4_t*>(src + i * kVec);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t d = (uint32_t)w[j];
            if constexpr (sizeof(T) == 4) {
                v[i * 4 + j] = __builtin_bit_cast(float, d);
            } else {
                v[i * 8 + 2 * j] = to_f32(__builtin_bit_cast(T, (uint16_t)(d & 0xffffu)));
                v[i * 8 + 2 * j + 1] = to_f32(__builtin_bit_cast(T, (uint16_t)(d >> 16)));
            }
        }
    }
}

template <typename T>
AA_DEV void store32(T* dst, const float (&v)[32]) {
    constexpr int kVec = 16 / sizeof(T);
#pragma unroll
    for (int i = 0; i < 32 / kVec; ++i) {
        i32x4_t w;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if constexpr (sizeof(T) == 4) {
                w[j] = __builtin_bit_cast(int, v[i * 4 + j]);
            } else {
                const uint32_t lo = __builtin_bit_cast(uint16_t, from_f32<T>(v[i * 8 + 2 * j]));
                const uint32_t hi = __builtin_bit_cast(uint16_t, from_f32<T>(v[i * 8 + 2 * j + 1]));
                w[j] = (int)(lo | (hi << 16));
            }
        }
        *reinterpret_cast<i32x4_t*>(dst + i * kVec) = w;
    }
}

// sum over the workgroup (every thread gets the total)
AA_DEV float block_sum(float v, float* red) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) t += red[w];
    return t;
}

// RMSNorm of one row of x2 (no quantisation): x2's elements need not form
// 32-blocks, so threads stride over elements and read the row twice
template <typename T>
AA_DEV void rms_row_plain(const RmsQuantParams& p, int row, float* red) {
    const T* x = reinterpret_cast<const T*>(p.x2) + row * p.x2_stride;
    const T* w = reinterpret_cast<const T*>(p.w2);
    T* out = reinterpret_cast<T*>(p.out2) + row * p.out2_stride;
    float ss = 0.f;
    for (int i = threadIdx.x; i < p.N2; i += kThreads) {
        const float v = to_f32(x[i]);
        ss += v * v;
    }
    const float nf = __builtin_amdgcn_rsqf(block_sum(ss, red) / (float)p.N2 + p.eps2);
    for (int i = threadIdx.x; i < p.N2; i += kThreads) out[i] = from_f32<T>(to_f32(x[i]) * nf * to_f32(w[i]));
}

// MAXB: blocks per thread kept in registers (1, 2 or 4: rows up to 8192,
// 16384, 32768 elements); fewer registers, more rows in flight per CU
template <typename T, bool OUT_FP8, int MAXB>
__global__ __launch_bounds__(kThreads) void rms_mx_quant_kernel(RmsQuantParams p) {
    __shared__ float red[kThreads / 64];
    if ((int)blockIdx.x >= p.M) {
        rms_row_plain<T>(p, (int)blockIdx.x - p.M, red);
        return;
    }
    const int row = blockIdx.x;
    const int nblk = p.N1 / 32;
    const T* x1 = reinterpret_cast<const T*>(p.x1) + row * p.x1_stride;
    const T* r1 = p.res1 ? reinterpret_cast<const T*>(p.res1) + row * p.res1_stride : nullptr;
    const T* w1 = reinterpret_cast<const T*>(p.w1);

    float v[MAXB][32];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < MAXB; ++i) {
        const int b = threadIdx.x + i * kThreads;
        if (b < nblk) {
            load32(x1 + b * 32, v[i]);
            if (r1) {
                float r[32];
                load32(r1 + b * 32, r);
#pragma unroll
                for (int e = 0; e < 32; ++e) v[i][e] += r[e];
                store32(reinterpret_cast<T*>(p.out_res1) + row * p.out_res1_stride + b * 32, v[i]);
            }
#pragma unroll
            for (int e = 0; e < 32; ++e) ss += v[i][e] * v[i][e];
        }
    }
    const float nf = __builtin_amdgcn_rsqf(block_sum(ss, red) / (float)p.N1 + p.eps1);

    constexpr uint32_t kEmax = OUT_FP8 ? 8u : 2u;
#pragma unroll
    for (int i = 0; i < MAXB; ++i) {
        const int b = threadIdx.x + i * kThreads;
        if (b < nblk) {
            float wv[32];
            load32(w1 + b * 32, wv);
            float amax = 0.f;
#pragma unroll
            for (int e = 0; e < 32; ++e) {
                v[i][e] = v[i][e] * nf * wv[e];
                amax = __builtin_fmaxf(amax, __builtin_fabsf(v[i][e]));
            }
            if (p.out1) store32(reinterpret_cast<T*>(p.out1) + row * p.out1_stride + b * 32, v[i]);
            const uint32_t byte = e8m0_byte<kEven>(amax, 0.f, 0.f, 0x200000u, kEmax);
            const float ds = __builtin_bit_cast(float, byte << 23);
            const bool hw = byte != 0u && byte != 255u;
            const float inv = inv_scale_from_byte(byte);
            if constexpr (OUT_FP8) {
                i32x4_t o[2];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    uint32_t w = 0;
                    if (hw) {
                        w = cvt_fp8_pair<float>(w, 0u, v[i][4 * k], v[i][4 * k + 1], ds, false);
                        w = cvt_fp8_pair<float>(w, 0u, v[i][4 * k + 2], v[i][4 * k + 3], ds, true);
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; ++j) w |= f32_to_e4m3(v[i][4 * k + j] * inv) << (8 * j);
                    }
                    o[k / 4][k % 4] = (int)w;
                }
                uint8_t* dst = p.q + row * p.q_stride + b * 32;
                *reinterpret_cast<i32x4_t*>(dst) = o[0];
                *reinterpret_cast<i32x4_t*>(dst + 16) = o[1];
            } else {
                i32x4_t o;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    uint32_t w = 0;
                    if (hw) {
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            w = cvt_fp4_pair<float>(w, 0u, v[i][8 * k + 2 * j], v[i][8 * k + 2 * j + 1], ds, j);
                    } else {
#pragma unroll
                        for (int j = 0; j < 8; ++j) w |= f32_to_e2m1(v[i][8 * k + j] * inv) << (4 * j);
                    }
                    o[k] = (int)w;
                }
                *reinterpret_cast<i32x4_t*>(p.q + row * p.q_stride + b * 16) = o;
            }
            if (p.shuffle)
                p.scale[scale_shuffle_idx(p.scale_n_pad, row, b)] = (uint8_t)byte;
            else
                p.scale[row * p.scale_stride + b] = (uint8_t)byte;
        }
    }
    // padding blocks of the row hold 127 (2^0), as the reference kernel writes
    if (p.pad_scale)
        for (int b = nblk + threadIdx.x; b < p.scale_n_pad; b += kThreads) {
            if (p.shuffle)
                p.scale[scale_shuffle_idx(p.scale_n_pad, row, b)] = 127;
            else
                p.scale[row * p.scale_stride + b] = 127;
        }
}

template <bool FP8, int MAXB>
void launch_blocks(int dt, const RmsQuantParams& p, unsigned grid, hipStream_t st) {
    if (dt == AITER_DTYPE_bf16)
        rms_mx_quant_kernel<__bf16, FP8, MAXB><<<grid, kThreads, 0, st>>>(p);
    else if (dt == AITER_DTYPE_fp16)
        rms_mx_quant_kernel<_Float16, FP8, MAXB><<<grid, kThreads, 0, st>>>(p);
    else
        rms_mx_quant_kernel<float, FP8, MAXB><<<grid, kThreads, 0, st>>>(p);
}

template <bool FP8>
void launch_typed(int dt, const RmsQuantParams& p, unsigned grid, hipStream_t st) {
    const int per_thread = (p.N1 / 32 + kThreads - 1) / kThreads;
    if (per_thread <= 1) launch_blocks<FP8, 1>(dt, p, grid, st);
    else if (per_thread <= 2) launch_blocks<FP8, 2>(dt, p, grid, st);
    else launch_blocks<FP8, kMaxBlocks>(dt, p, grid, st);
}

}  // namespace

extern "C" {

int fused_rms_mx_quant(aiter_tensor_t* x1, aiter_tensor_t* w1, float eps1, aiter_tensor_t* x2,
                       aiter_tensor_t* w2, float eps2, aiter_tensor_t* res1, aiter_tensor_t* out_q,
                       aiter_tensor_t* out_scale, aiter_tensor_t* out1, aiter_tensor_t* out2,
                       aiter_tensor_t* out_res1, int shuffle, int pad_scale, aiter_stream_t stream) {
    using namespace aiter_amd;
    return safe_call([&] {
        check_tensor(x1, "x1", 2);
        check_tensor(w1, "x1_weight");
        check_tensor(out_q, "out_q", 2);
        check_tensor(out_scale, "out_scale");
        DeviceGuard g(x1->device_id);
        const int dt = x1->dtype;
        AA_CHECK(dt == AITER_DTYPE_bf16 || dt == AITER_DTYPE_fp16 || dt == AITER_DTYPE_fp32,
                 "x1 must be bf16/fp16/fp32, got ", dtype_name(dt));
        const int64_t M = rows_2d(x1), N1 = cols_2d(x1);
        AA_CHECK(N1 % 32 == 0, "x1 last dim ", N1, " must be a multiple of 32");
        AA_CHECK(N1 / 32 <= (int64_t)kMaxBlocks * kThreads, "x1 last dim ", N1, " exceeds ", kMaxBlocks * kThreads * 32);
        AA_CHECK(w1->dtype == dt && (int64_t)w1->numel == N1, "x1_weight must be [N1] of x1's dtype");
        const int64_t esz = dtype_size(dt);
        auto aligned = [&](const aiter_tensor_t* t, const char* nm) {
            AA_CHECK(((uintptr_t)t->ptr & 15) == 0 && (row_stride_2d(t, nm) * esz) % 16 == 0,
                     nm, " rows must be 16-byte aligned");
        };
        aligned(x1, "x1");
        AA_CHECK(((uintptr_t)w1->ptr & 15) == 0, "x1_weight must be 16-byte aligned");
        const bool fp8 = out_q->dtype == AITER_DTYPE_fp8;
        AA_CHECK(fp8 || is_byte_type(out_q->dtype), "out_q must be u8 (e2m1 pairs) or fp8");
        AA_CHECK(rows_2d(out_q) == M && cols_2d(out_q) == (fp8 ? N1 : N1 / 2), "out_q must be [M, ",
                 fp8 ? N1 : N1 / 2, "]");
        AA_CHECK(((uintptr_t)out_q->ptr & 15) == 0 && row_stride_2d(out_q, "out_q") % 16 == 0,
                 "out_q rows must be 16-byte aligned");
        AA_CHECK(is_byte_type(out_scale->dtype), "out_scale must be u8 / e8m0");

        RmsQuantParams p{};
        p.x1 = x1->ptr;
        p.w1 = w1->ptr;
        p.M = (int)M;
        p.N1 = (int)N1;
        p.eps1 = eps1;
        p.eps2 = eps2;
        p.x1_stride = row_stride_2d(x1, "x1");
        p.q = static_cast<uint8_t*>(out_q->ptr);
        p.q_stride = row_stride_2d(out_q, "out_q");
        p.scale = static_cast<uint8_t*>(out_scale->ptr);
        p.shuffle = shuffle != 0;
        p.pad_scale = pad_scale != 0;
        const int nblk = (int)(N1 / 32);
        p.scale_n_pad = (p.shuffle || p.pad_scale) ? (nblk + 7) / 8 * 8 : nblk;
        if (p.shuffle) {
            AA_CHECK((int64_t)out_scale->numel >= (M + 255) / 256 * 256 * (int64_t)p.scale_n_pad,
                     "shuffled scale needs [pad256(M), pad8(N1/32)] bytes");
        } else {
            AA_CHECK(rows_2d(out_scale) >= M && cols_2d(out_scale) >= p.scale_n_pad,
                     "out_scale must be at least [M, ", p.scale_n_pad, "]");
            p.scale_stride = row_stride_2d(out_scale, "out_scale");
        }
        auto same_shape = [&](const aiter_tensor_t* t, const char* nm, int64_t cols) {
            check_tensor(t, nm, 2);
            AA_CHECK(t->dtype == dt && rows_2d(t) == M && cols_2d(t) == cols, nm, " must be [M, ", cols,
                     "] of x1's dtype");
            aligned(t, nm);
        };
        if (res1) {
            same_shape(res1, "res1", N1);
            AA_CHECK(out_res1, "res1 needs out_res1");
            same_shape(out_res1, "out_res1", N1);
            p.res1 = res1->ptr;
            p.res1_stride = row_stride_2d(res1, "res1");
            p.out_res1 = out_res1->ptr;
            p.out_res1_stride = row_stride_2d(out_res1, "out_res1");
        }
        if (out1) {
            same_shape(out1, "out1", N1);
            p.out1 = out1->ptr;
            p.out1_stride = row_stride_2d(out1, "out1");
        }
        unsigned grid = (unsigned)M;
        if (x2) {
            check_tensor(x2, "x2", 2);
            AA_CHECK(x2->dtype == dt && rows_2d(x2) == M, "x2 must be [M, N2] of x1's dtype");
            AA_CHECK(w2 && w2->dtype == dt && (int64_t)w2->numel == cols_2d(x2), "x2_weight must be [N2]");
            AA_CHECK(out2, "x2 needs out2");
            p.N2 = (int)cols_2d(x2);
            check_tensor(out2, "out2", 2);
            AA_CHECK(out2->dtype == dt && rows_2d(out2) == M && cols_2d(out2) == p.N2,
                     "out2 must be [M, N2] of x1's dtype");
            AA_CHECK(p.N2 > 0 && x2->strides[x2->ndim - 1] == 1 && out2->strides[out2->ndim - 1] == 1 &&
                     w2->strides[w2->ndim - 1] == 1, "x2, x2_weight and out2 need unit inner stride");
            p.x2 = x2->ptr;
            p.w2 = w2->ptr;
            p.x2_stride = row_stride_2d(x2, "x2");
            p.out2 = out2->ptr;
            p.out2_stride = row_stride_2d(out2, "out2");
            grid = (unsigned)(2 * M);
        }
        if (M == 0) return;
        const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
        if (fp8) launch_typed<true>(dt, p, grid, st);
        else launch_typed<false>(dt, p, grid, st);
        AA_HIP(hipGetLastError());
    });
}

}  // extern "C"
