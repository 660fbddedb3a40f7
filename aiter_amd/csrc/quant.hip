// Per-1x32 MX activation/weight quantisers (MXFP4 e2m1 / MXFP8 e4m3fn with
// e8m0 block scales) for gfx950.
//
// The plain quantiser gives each 32-element block to the four lanes of a
// quad: lane q reads elements 8q .. 8q+7 with 16-byte loads (so one load
// instruction of a wave reads 1 KiB of contiguous input), the quad exchanges
// its partial amax, every lane derives the e8m0 byte, converts its 8 values
// and writes 4 B (fp4) or 8 B (fp8), and lane 0 the scale byte.  The sorted
// MoE quantiser keeps one thread per block.  The work is HBM-bound: 64 B in
// / 17 B out per block for bf16 -> fp4.
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

// Quantises the 32 elements at src (16-byte aligned): returns the e8m0 byte
// and the packed codes (fp4: o[0]; fp8: o[0], o[1]).
template <typename InT, bool OUT_FP8, int MODE>
AA_DEV uint32_t quant_block32(const QuantParams& p, const InT* src, i32x4_t (&o)[2]) {
    constexpr int kVec = 16 / sizeof(InT);  // elements per 16-byte load
    float v[32];
    uint32_t raw[16];   // 16-bit inputs: the loaded element pairs (unused for f32)
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
    if constexpr (!OUT_FP8) {
        return quant32_fp4<InT, MODE>(v, raw, p.amax_floor, p.inv_max_pos, p.inv_max_pow2, p.even_add, p.emax,
                                      o[0]);
    } else {
        float amax = p.amax_floor;
#pragma unroll
        for (int i = 0; i < 32; ++i) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[i]));
        const uint32_t byte = e8m0_byte<MODE>(amax, p.inv_max_pos, p.inv_max_pow2, p.even_add, p.emax);
        const float inv = inv_scale_from_byte(byte);
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
        return byte;
    }
}

// max of a float over the four lanes of a quad (lanes 4i .. 4i+3), by two
// DPP quad permutes (xor 1, xor 2); a max is exact in any order
AA_DEV float quad_max(float a) {
    a = __builtin_fmaxf(a, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, a),
                                                                                   0xB1, 0xF, 0xF, false)));
    a = __builtin_fmaxf(a, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, a),
                                                                                   0x4E, 0xF, 0xF, false)));
    return a;
}

// The 16-byte words a lane loads for its quarter of a block: elements
// 8q .. 8q+7 (one word for 16-bit inputs, two for f32).
template <typename InT>
struct QuarterIn {
    i32x4_t w[sizeof(InT) == 4 ? 2 : 1];
};

template <typename InT>
AA_DEV void load_quarter(const InT* src, int q, QuarterIn<InT>& in) {
#pragma unroll
    for (int h = 0; h < (sizeof(InT) == 4 ? 2 : 1); ++h)
        in.w[h] = *reinterpret_cast<const i32x4_t*>(src + 8 * q + 4 * h);
}

// Quarter q of a 32-element block, held by lane q of the quad that shares
// the block: the block's amax comes from the quad, so each lane derives the
// same e8m0 byte and converts its 8 elements exactly as quant_block32
// converts them.  Codes: fp4 o[0] (8 nibbles), fp8 o[0], o[1] (8 bytes).
template <typename InT, bool OUT_FP8, int MODE>
AA_DEV uint32_t quant_quarter(const QuantParams& p, const QuarterIn<InT>& in, uint32_t (&o)[2]) {
    float v[8];
    uint32_t raw[4];   // 16-bit inputs: the loaded element pairs
    if constexpr (sizeof(InT) == 4) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = in.w[h][j];
                v[4 * h + j] = __builtin_bit_cast(float, e);
            }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t d = (uint32_t)in.w[0][j];
            raw[j] = d;
            if constexpr (std::is_same<InT, _Float16>::value) {
                v[2 * j] = (float)__builtin_bit_cast(_Float16, (uint16_t)(d & 0xffffu));
                v[2 * j + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(d >> 16));
            } else {
                v[2 * j] = __builtin_bit_cast(float, d << 16);
                v[2 * j + 1] = __builtin_bit_cast(float, d & 0xffff0000u);
            }
        }
    }
    float amax = p.amax_floor;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[i]));
    amax = quad_max(amax);
    const uint32_t byte = e8m0_byte<MODE>(amax, p.inv_max_pos, p.inv_max_pow2, p.even_add, p.emax);
    const float inv = inv_scale_from_byte(byte);
    const bool normal = byte != 0u && byte != 255u;
    const float ds = __builtin_bit_cast(float, byte << 23);
    if constexpr (!OUT_FP8) {
        uint32_t w = 0;
        if (normal) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (sizeof(InT) == 2)
                    w = cvt_fp4_pair<InT>(w, raw[j], 0.f, 0.f, ds, j);
                else
                    w = cvt_fp4_pair<float>(w, 0u, v[2 * j], v[2 * j + 1], ds, j);
            }
        } else {
            // scale byte 0 (2^-127, a subnormal f32) or 255 (NaN)
#pragma unroll
            for (int j = 0; j < 8; ++j) w |= f32_to_e2m1(v[j] * inv) << (4 * j);
        }
        o[0] = w;
        o[1] = 0;
    } else {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            uint32_t w = 0;
            if (normal) {
                if constexpr (sizeof(InT) == 2) {
                    w = cvt_fp8_pair<InT>(w, raw[2 * i], 0.f, 0.f, ds, false);
                    w = cvt_fp8_pair<InT>(w, raw[2 * i + 1], 0.f, 0.f, ds, true);
                } else {
                    w = cvt_fp8_pair<float>(w, 0u, v[4 * i], v[4 * i + 1], ds, false);
                    w = cvt_fp8_pair<float>(w, 0u, v[4 * i + 2], v[4 * i + 3], ds, true);
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) w |= f32_to_e4m3(v[i * 4 + j] * inv) << (8 * j);
            }
            o[i] = w;
        }
    }
    return byte;
}

// Four lanes per 32-element block (lane q: elements 8q .. 8q+7), so that one
// load instruction of a wave reads 16 consecutive blocks (1 KiB of bf16) and
// one store writes 256 B of fp4 codes; each wave takes 16*kQuantUnroll
// consecutive blocks, all loads issued before converting.  A quad (4
// consecutive lanes) always shares one block, so the quad exchange never
// meets an exited lane.  Measured cold at 8192 x 8192 bf16: one thread per
// block 41.5 us, a quad per block 37.0-38.3 us, a quad per block with 4
// blocks per lane 43.7 us.
constexpr int kQuantUnroll = 1;

template <typename InT, bool OUT_FP8, int MODE>
__global__ __launch_bounds__(256) void mx_quant_kernel(QuantParams p) {
    const int lane = threadIdx.x & 63;
    const int q = lane & 3;
    const int64_t blk0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * (16 * kQuantUnroll) + (lane >> 2);
    int64_t rows = p.rows;
    if (p.num_rows) rows = (int64_t)(*p.num_rows) * p.num_rows_factor;
    QuarterIn<InT> in[kQuantUnroll];
    int64_t xs[kQuantUnroll];
    int ys[kQuantUnroll];
#pragma unroll
    for (int u = 0; u < kQuantUnroll; ++u) {
        const int64_t blk = blk0 + 16 * u;
        xs[u] = blk / p.scale_n_pad;
        ys[u] = (int)(blk % p.scale_n_pad);
        if (xs[u] < rows && xs[u] < p.cover_rows && ys[u] < p.scale_n)
            load_quarter<InT>(reinterpret_cast<const InT*>(p.in) + xs[u] * p.in_stride + (int64_t)ys[u] * 32, q,
                              in[u]);
    }
#pragma unroll
    for (int u = 0; u < kQuantUnroll; ++u) {
        const int64_t x = xs[u];
        const int y = ys[u];
        if (x >= p.cover_rows) continue;
        if (!(x < rows && y < p.scale_n)) {
            // padding of the (Triton-layout) shuffled scale buffer is written as zero
            if (p.zero_pad && q == 0) p.scale[scale_shuffle_idx(p.scale_n_pad, (int)x, y)] = 0;
            continue;
        }
        uint32_t o[2];
        const uint32_t byte = quant_quarter<InT, OUT_FP8, MODE>(p, in[u], o);
        if constexpr (OUT_FP8) {
            typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
            *reinterpret_cast<u32x2_t*>(p.out + x * p.out_stride + (int64_t)y * 32 + 8 * q) = u32x2_t{o[0], o[1]};
        } else {
            int64_t off;
            if (p.shuffle_weight) {
                // shuffle_weight((16,16)) position of bytes [16y, 16y+16) of row x
                // (aiter/ops/shuffle.py:192-204; fused form csrc/kernels/quant_mxfp4.cu:177-183)
                off = (x >> 4) * 16 * p.out_stride + (x & 15) * 16 + (int64_t)(y >> 1) * 512 + (y & 1) * 256;
            } else {
                off = x * p.out_stride + (int64_t)y * 16;
            }
            *reinterpret_cast<uint32_t*>(p.out + off + 4 * q) = o[0];
        }
        if (q == 0) {
            if (p.shuffle_scale)
                p.scale[scale_shuffle_idx(p.scale_n_pad, (int)x, y)] = (uint8_t)byte;
            else
                p.scale[x * p.scale_stride + y] = (uint8_t)byte;
        }
    }
}

template <typename InT, bool OUT_FP8>
void launch_mode(int mode, const QuantParams& p, int64_t nthreads, hipStream_t st) {
    // nthreads = blocks; 4 lanes per block, 16 * kQuantUnroll blocks per wave
    const dim3 grid((unsigned)((nthreads + 64 * kQuantUnroll - 1) / (64 * kQuantUnroll)));
    switch (mode) {
        case kRoundDown: mx_quant_kernel<InT, OUT_FP8, kRoundDown><<<grid, 256, 0, st>>>(p); break;
        case kRoundUp: mx_quant_kernel<InT, OUT_FP8, kRoundUp><<<grid, 256, 0, st>>>(p); break;
        case kEven: mx_quant_kernel<InT, OUT_FP8, kEven><<<grid, 256, 0, st>>>(p); break;
        case kCeil: mx_quant_kernel<InT, OUT_FP8, kCeil><<<grid, 256, 0, st>>>(p); break;
        default: aiter_amd::fail("quant", "round_mode must be 0..3, got ", mode);
    }
}

// ---- MoE: rows named by a sorted routing list, scale bytes in sorted order ----
// Sorted position x holds entry sorted_ids[x] = slot << 24 | token; its input
// row is token (stage 1: one row per token) or token * topk + slot (stage 2:
// one row per routed pair).  Scale byte (x, block) goes to the shuffled
// [pad32(len), pad8(K/32)] layout at row x, so that a GEMM over the sorted
// list reads its A scales in row order.  One workgroup (or thread, for the
// byte sort) per 32 sorted positions; groups at or past num_valid_ids[0] (a
// multiple of the row block) exit at once and leave their bytes unwritten, as
// the GEMM never reads them.  Padding positions inside the list (token >=
// token count) and padding columns get scale byte 0.
struct SortQuant {
    const int* sorted_ids;
    const int* num_valid;
    const float* sorted_w;    // optional: a zero routing weight writes a zero row
    int64_t sorted_rows;      // positions covered (pad32 of the sorted list)
    int token_num, topk;
};

AA_DEV int64_t sorted_source_row(const SortQuant& s, int64_t x, int& valid) {
    const int nv = *s.num_valid;
    const int id = x < nv ? s.sorted_ids[x] : s.token_num;
    const int token = id & 0xffffff, slot = (int)((unsigned)id >> 24);
    valid = token < s.token_num && (s.topk == 1 || slot < s.topk);
    return s.topk == 1 ? (int64_t)token : (int64_t)token * s.topk + slot;
}

// fused quant + sort (csrc/kernels/quant_kernels.cu:1733-1880): RoundUp e8m0
// from the running max 1e-10, one thread per (sorted position, 32-block);
// workgroup (x, y) covers sorted positions 32x.. and scale columns 32y..
template <typename InT, bool OUT_FP8>
__global__ __launch_bounds__(256) void mx_quant_sorted_kernel(QuantParams p, SortQuant s) {
    const int64_t g0 = (int64_t)blockIdx.x * 32;
    const int nv = *s.num_valid;
    if (g0 >= nv) return;
    // the group's 32 input rows, resolved once (not one dependent load per item)
    __shared__ int64_t rows[32];
    __shared__ int valid_of[32];
    if (threadIdx.x < 32) {
        int v;
        rows[threadIdx.x] = sorted_source_row(s, g0 + threadIdx.x, v);
        valid_of[threadIdx.x] = v;
    }
    __syncthreads();
    // columns split over gridDim.y in runs of 32 blocks: a few items per
    // thread instead of a long serial loop at large K
    const int y0 = blockIdx.y * 32;
    const int ny = min(32, p.scale_n_pad - y0);
    const int items = 32 * ny;
    for (int it = threadIdx.x; it < items; it += 256) {
        const int xr = it / ny;
        const int64_t x = g0 + xr;
        const int y = y0 + it % ny;
        const int valid = valid_of[xr];
        const int64_t row = rows[xr];
        uint8_t* sc = p.scale + scale_shuffle_idx(p.scale_n_pad, (int)x, y);
        if (!valid || y >= p.scale_n) {
            *sc = 0;
            continue;
        }
        constexpr int OB = OUT_FP8 ? 32 : 16;   // output bytes per block
        uint8_t* dst = p.out + row * p.out_stride + (int64_t)y * OB;
        i32x4_t o[2] = {i32x4_t{0, 0, 0, 0}, i32x4_t{0, 0, 0, 0}};
        uint32_t byte = 0;
        if (!(s.sorted_w && s.sorted_w[x] == 0.0f)) {
            const InT* src = reinterpret_cast<const InT*>(p.in) + row * p.in_stride + (int64_t)y * 32;
            byte = quant_block32<InT, OUT_FP8, kRoundUp>(p, src, o);
        }
        *reinterpret_cast<i32x4_t*>(dst) = o[0];
        if constexpr (OUT_FP8) *reinterpret_cast<i32x4_t*>(dst + 16) = o[1];
        *sc = (uint8_t)byte;
    }
}

// byte sort of per-row scales (csrc/kernels/quant_kernels.cu mxfp4_moe_sort):
// plain [rows, K/32] -> sorted shuffled layout.  Byte (x = 32g + xr, y = 8y8
// + yy) sits at g * 32 * pad8 + y8 * 256 + dword (yy % 4) * 16 + xr % 16, byte
// (yy / 4) * 2 + xr / 16 (mx_scale_shuffle_idx).  Thread (g, y8, h) owns the
// dwords with xr % 16 in [8h, 8h + 8): rows 8h.. and 16 + 8h.. of the group,
// four 32-byte runs of the 256-byte block, built in registers.
__global__ __launch_bounds__(256) void mx_scale_sort_kernel(const uint8_t* scale, int64_t scale_stride, uint8_t* out,
                                                            SortQuant s, int scale_n, int scale_n_pad) {
    const int y8n = scale_n_pad / 8;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int h = (int)(gid & 1);
    const int64_t g = (gid >> 1) / y8n;
    const int y8 = (int)((gid >> 1) % y8n);
    if (g * 32 >= s.sorted_rows || g * 32 >= *s.num_valid) return;
    const bool whole = (scale_stride % 8 == 0) && (y8 * 8 + 8 <= scale_n);
    uint32_t o[32];
#pragma unroll
    for (int k = 0; k < 32; ++k) o[k] = 0;
#pragma unroll
    for (int xs = 0; xs < 16; ++xs) {
        const int xr = (xs < 8) ? 8 * h + xs : 16 + 8 * h + (xs - 8);
        int valid;
        const int64_t row = sorted_source_row(s, g * 32 + xr, valid);
        if (!valid) continue;
        const uint8_t* src = scale + row * scale_stride + y8 * 8;
        uint32_t lo = 0, hi = 0;
        if (whole) {
            const uint2 v = *reinterpret_cast<const uint2*>(src);
            lo = v.x;
            hi = v.y;
        } else {
#pragma unroll
            for (int yy = 0; yy < 8; ++yy) {
                const uint32_t b = (y8 * 8 + yy < scale_n) ? src[yy] : 0u;
                if (yy < 4) lo |= b << (8 * yy);
                else hi |= b << (8 * (yy - 4));
            }
        }
#pragma unroll
        for (int yy = 0; yy < 8; ++yy) {
            const uint32_t b = ((yy < 4 ? lo : hi) >> (8 * (yy & 3))) & 0xffu;
            o[(yy & 3) * 8 + (xs & 7)] |= b << (8 * ((yy >> 2) * 2 + (xs >> 3)));
        }
    }
    uint8_t* dst = out + g * scale_n_pad * 32 + (int64_t)y8 * 256 + h * 32;
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) {
        *reinterpret_cast<i32x4_t*>(dst + k4 * 64) =
            i32x4_t{(int)o[8 * k4], (int)o[8 * k4 + 1], (int)o[8 * k4 + 2], (int)o[8 * k4 + 3]};
        *reinterpret_cast<i32x4_t*>(dst + k4 * 64 + 16) =
            i32x4_t{(int)o[8 * k4 + 4], (int)o[8 * k4 + 5], (int)o[8 * k4 + 6], (int)o[8 * k4 + 7]};
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

int fused_dynamic_mx_quant_moe_sort_hip(aiter_tensor_t* out, aiter_tensor_t* scales, aiter_tensor_t* input,
                                        aiter_tensor_t* sorted_ids, aiter_tensor_t* num_valid_ids, int token_num,
                                        int block_m, int group_size, aiter_tensor_t* sorted_weights,
                                        aiter_stream_t stream) {
    using namespace aiter_amd;
    return safe_call([&] {
        AA_CHECK(group_size == 32, "only group_size 32 (MX) is implemented, got ", group_size);
        (void)block_m;
        check_tensor(out, "out");
        check_tensor(scales, "scales");
        check_tensor(input, "input");
        check_tensor(sorted_ids, "sorted_ids");
        check_tensor(num_valid_ids, "num_valid_ids");
        DeviceGuard g(input->device_id);
        const int in_dt = input->dtype;
        AA_CHECK(in_dt == AITER_DTYPE_bf16 || in_dt == AITER_DTYPE_fp16 || in_dt == AITER_DTYPE_fp32,
                 "input must be bf16/fp16/fp32");
        const bool fp8 = out->dtype == AITER_DTYPE_fp8;
        AA_CHECK(fp8 || out->dtype == AITER_DTYPE_fp4x2 || out->dtype == AITER_DTYPE_u8, "out must be fp4x2 or fp8");
        AA_CHECK(sorted_ids->dtype == AITER_DTYPE_i32 && num_valid_ids->dtype == AITER_DTYPE_i32,
                 "sorted_ids / num_valid_ids must be int32");
        const int64_t rows = rows_2d(input), cols = cols_2d(input);
        AA_CHECK(cols % 32 == 0, "input columns must be a multiple of 32");
        AA_CHECK(token_num > 0 && rows % token_num == 0, "input rows ", rows, " must be a multiple of token_num ",
                 token_num);
        AA_CHECK(input->strides[input->ndim - 1] == 1 && ((uintptr_t)input->ptr & 15) == 0,
                 "input must have unit column stride and 16-byte alignment");
        const int64_t in_stride = input->ndim >= 2 ? input->strides[input->ndim - 2] : cols;
        AA_CHECK(in_stride % (16 / dtype_size(in_dt)) == 0, "input row stride must keep 16-byte alignment");
        const int64_t out_cols = fp8 ? cols : cols / 2;
        AA_CHECK(rows_2d(out) == rows && cols_2d(out) == out_cols && out->strides[out->ndim - 1] == 1,
                 "out must be [", rows, ", ", out_cols, "]");
        const int64_t out_stride = out->ndim >= 2 ? out->strides[out->ndim - 2] : out_cols;
        AA_CHECK(out_stride % 16 == 0 && ((uintptr_t)out->ptr & 15) == 0, "out rows must be 16-byte aligned");
        const int scale_n = (int)(cols / 32), scale_n_pad = (scale_n + 7) / 8 * 8;
        const int64_t sorted_rows = ((int64_t)sorted_ids->numel + 31) / 32 * 32;
        AA_CHECK((int64_t)scales->numel >= sorted_rows * scale_n_pad, "scales needs [pad32(len(sorted_ids)), ",
                 scale_n_pad, "] bytes");
        if (sorted_weights) {
            AA_CHECK(sorted_weights->dtype == AITER_DTYPE_fp32 && sorted_weights->numel >= sorted_ids->numel,
                     "sorted_weights must be float32 with len(sorted_ids) entries");
        }
        QuantParams p{};
        p.in = input->ptr;
        p.out = static_cast<uint8_t*>(out->ptr);
        p.scale = static_cast<uint8_t*>(scales->ptr);
        p.in_stride = in_stride;
        p.out_stride = out_stride;
        p.scale_n = scale_n;
        p.scale_n_pad = scale_n_pad;
        p.cols = (int)cols;
        p.inv_max_pos = fp8 ? 1.0f / 448.0f : 1.0f / 6.0f;
        p.inv_max_pow2 = fp8 ? 1.0f / 256.0f : 0.25f;
        p.emax = fp8 ? 8 : 2;
        p.amax_floor = 1e-10f;   // csrc/kernels/quant_kernels.cu:1837
        SortQuant s{};
        s.sorted_ids = static_cast<const int*>(sorted_ids->ptr);
        s.num_valid = static_cast<const int*>(num_valid_ids->ptr);
        s.sorted_w = sorted_weights ? static_cast<const float*>(sorted_weights->ptr) : nullptr;
        s.sorted_rows = sorted_rows;
        s.token_num = token_num;
        s.topk = (int)(rows / token_num);
        const dim3 grid((unsigned)(sorted_rows / 32), (unsigned)((scale_n_pad + 31) / 32));
        hipStream_t st = reinterpret_cast<hipStream_t>(stream);
        if (in_dt == AITER_DTYPE_bf16) {
            if (fp8) mx_quant_sorted_kernel<uint16_t, true><<<grid, 256, 0, st>>>(p, s);
            else mx_quant_sorted_kernel<uint16_t, false><<<grid, 256, 0, st>>>(p, s);
        } else if (in_dt == AITER_DTYPE_fp16) {
            if (fp8) mx_quant_sorted_kernel<_Float16, true><<<grid, 256, 0, st>>>(p, s);
            else mx_quant_sorted_kernel<_Float16, false><<<grid, 256, 0, st>>>(p, s);
        } else {
            if (fp8) mx_quant_sorted_kernel<float, true><<<grid, 256, 0, st>>>(p, s);
            else mx_quant_sorted_kernel<float, false><<<grid, 256, 0, st>>>(p, s);
        }
        AA_HIP(hipGetLastError());
    });
}

int mxfp4_moe_sort_hip(aiter_tensor_t* out_scale, aiter_tensor_t* scale, aiter_tensor_t* sorted_ids,
                       aiter_tensor_t* num_valid_ids, int token_num, int cols, aiter_stream_t stream) {
    using namespace aiter_amd;
    return safe_call([&] {
        check_tensor(out_scale, "out_scale");
        check_tensor(scale, "scale", 2);
        check_tensor(sorted_ids, "sorted_ids");
        check_tensor(num_valid_ids, "num_valid_ids");
        DeviceGuard g(scale->device_id);
        AA_CHECK(is_byte_type(scale->dtype) && is_byte_type(out_scale->dtype), "scales must be e8m0/u8");
        AA_CHECK(sorted_ids->dtype == AITER_DTYPE_i32 && num_valid_ids->dtype == AITER_DTYPE_i32,
                 "sorted_ids / num_valid_ids must be int32");
        const int scale_n = (cols + 31) / 32, scale_n_pad = (scale_n + 7) / 8 * 8;
        const int64_t rows = rows_2d(scale);
        AA_CHECK(token_num > 0 && rows % token_num == 0, "scale rows ", rows, " must be a multiple of token_num");
        AA_CHECK(cols_2d(scale) >= scale_n && scale->strides[scale->ndim - 1] == 1, "scale must be [rows, ",
                 scale_n, "]");
        const int64_t sorted_rows = ((int64_t)sorted_ids->numel + 31) / 32 * 32;
        AA_CHECK((int64_t)out_scale->numel >= sorted_rows * scale_n_pad, "out_scale needs [pad32(len(sorted_ids)), ",
                 scale_n_pad, "] bytes");
        SortQuant s{};
        s.sorted_ids = static_cast<const int*>(sorted_ids->ptr);
        s.num_valid = static_cast<const int*>(num_valid_ids->ptr);
        s.sorted_rows = sorted_rows;
        s.token_num = token_num;
        s.topk = (int)(rows / token_num);
        const int64_t nthreads = sorted_rows / 32 * (scale_n_pad / 8) * 2;
        mx_scale_sort_kernel<<<(unsigned)((nthreads + 255) / 256), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
            static_cast<const uint8_t*>(scale->ptr), scale->strides[scale->ndim - 2], static_cast<uint8_t*>(out_scale->ptr),
            s, scale_n, scale_n_pad);
        AA_HIP(hipGetLastError());
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
