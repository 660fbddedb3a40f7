// HBM read-rate calibration: a plain streaming read with nothing else in the
// kernel, the attainable rate that the bandwidth-bound GEMMs (decode shapes)
// are compared against at the same byte count.  Not an operator: no
// counterpart in the reference.
#include "common.h"
#include "mfma32.h"

namespace aiter_amd {
namespace {

constexpr int kUnroll = 4;

// grid-stride over 16-byte words, kUnroll independent loads per thread in
// flight; the xor of everything read is kept live by a store that only a
// 1-in-2^32 value triggers
__global__ __launch_bounds__(256) void stream_read_kernel(const i32x4_t* __restrict__ src, int64_t n16, int* sink) {
    i32x4_t acc = {0, 0, 0, 0};
    const int64_t stride = (int64_t)gridDim.x * 256 * kUnroll;
    for (int64_t i = (int64_t)blockIdx.x * 256 * kUnroll + threadIdx.x; i < n16; i += stride) {
        i32x4_t v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t j = i + (int64_t)u * 256;
            v[u] = j < n16 ? __builtin_nontemporal_load(src + j) : i32x4_t{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) acc ^= v[u];
    }
    if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x5eed1e55) sink[0] = 1;
}

// The same read with its launch shape and cache policy as parameters: U
// loads per thread in flight, B threads per workgroup, buffer loads with
// cache-policy bits POL (gfx950: bit 0 sc0, bit 1 nt, bit 4 sc1; POL < 0:
// __builtin_nontemporal_load, as stream_read_kernel).  NOLOAD: an empty
// kernel of the same grid (the launch floor of a graph-replayed call).
template <int U, int B, int POL, bool NOLOAD>
__global__ __launch_bounds__(B) void stream_read_cfg_kernel(const i32x4_t* __restrict__ src, int64_t n16, int* sink) {
    if constexpr (NOLOAD) {
        if (n16 < 0) sink[0] = 1;
        return;
    } else {
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(src, n16 * 16 < (1LL << 31) ? n16 * 16 : 0);
        const bool buffered = POL >= 0 && n16 * 16 < (1LL << 31);
        i32x4_t acc = {0, 0, 0, 0};
        const int64_t stride = (int64_t)gridDim.x * B * U;
        for (int64_t i = (int64_t)blockIdx.x * B * U + threadIdx.x; i < n16; i += stride) {
            i32x4_t v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int64_t j = i + (int64_t)u * B;
                if (buffered)   // past the end: the range check returns zeros
                    v[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(j * 16), 0, POL < 0 ? 0 : POL);
                else
                    v[u] = j < n16 ? __builtin_nontemporal_load(src + j) : i32x4_t{0, 0, 0, 0};
            }
#pragma unroll
            for (int u = 0; u < U; ++u) acc ^= v[u];
        }
        if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x5eed1e55) sink[0] = 1;
    }
}

using CalibFn = void (*)(const i32x4_t*, int64_t, int*, int, hipStream_t);

template <int U, int B, int POL, bool NOLOAD = false>
void launch_cfg(const i32x4_t* src, int64_t n16, int* sink, int grid, hipStream_t st) {
    stream_read_cfg_kernel<U, B, POL, NOLOAD><<<grid, B, 0, st>>>(src, n16, sink);
}

template <int U, int B>
CalibFn pick_policy(int pol) {
    switch (pol) {
        case -1: return launch_cfg<U, B, -1>;
        case 0: return launch_cfg<U, B, 0>;
        case 1: return launch_cfg<U, B, 1>;
        case 2: return launch_cfg<U, B, 2>;
        case 3: return launch_cfg<U, B, 3>;
        case 16: return launch_cfg<U, B, 16>;
        case 17: return launch_cfg<U, B, 17>;
        case 18: return launch_cfg<U, B, 18>;
        case 19: return launch_cfg<U, B, 19>;
        default: return nullptr;
    }
}

template <int U>
CalibFn pick_block(int block, int pol) {
    switch (block) {
        case 64: return pick_policy<U, 64>(pol);
        case 128: return pick_policy<U, 128>(pol);
        case 256: return pick_policy<U, 256>(pol);
        case 512: return pick_policy<U, 512>(pol);
        case 1024: return pick_policy<U, 1024>(pol);
        default: return nullptr;
    }
}

CalibFn pick_cfg(int unroll, int block, int pol) {
    if (pol == -2) return block == 256 ? launch_cfg<1, 256, 0, true> : nullptr;
    switch (unroll) {
        case 1: return pick_block<1>(block, pol);
        case 2: return pick_block<2>(block, pol);
        case 4: return pick_block<4>(block, pol);
        case 8: return pick_block<8>(block, pol);
        default: return nullptr;
    }
}

}  // namespace
}  // namespace aiter_amd

using namespace aiter_amd;

extern "C" {

int hbm_stream_read(aiter_tensor_t* src, aiter_tensor_t* sink, int grid, aiter_stream_t stream) {
    return safe_call([&] {
        check_tensor(src, "src", 1);
        check_tensor(sink, "sink", 1);
        DeviceGuard g(src->device_id);
        AA_CHECK(src->ndim == 1 && src->strides[0] == 1, "hbm_stream_read: src must be a contiguous 1-D tensor");
        AA_CHECK(sink->dtype == AITER_DTYPE_i32 && sink->numel >= 1, "hbm_stream_read: sink must hold one int32");
        const int64_t bytes = (int64_t)src->numel * dtype_size(src->dtype);
        AA_CHECK(bytes % 16 == 0 && ((uintptr_t)src->ptr & 15) == 0,
                 "hbm_stream_read: src must be 16-byte aligned and a multiple of 16 bytes");
        AA_CHECK(grid > 0 && grid <= (1 << 20), "hbm_stream_read: grid out of range: ", grid);
        if (bytes == 0) return;
        stream_read_kernel<<<grid, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
            static_cast<const i32x4_t*>(src->ptr), bytes / 16, static_cast<int*>(sink->ptr));
        AA_HIP(hipGetLastError());
    });
}

int hbm_stream_read_cfg(aiter_tensor_t* src, aiter_tensor_t* sink, int grid, int block, int unroll, int policy,
                        aiter_stream_t stream) {
    return safe_call([&] {
        check_tensor(src, "src", 1);
        check_tensor(sink, "sink", 1);
        DeviceGuard g(src->device_id);
        AA_CHECK(src->ndim == 1 && src->strides[0] == 1, "hbm_stream_read_cfg: src must be a contiguous 1-D tensor");
        AA_CHECK(sink->dtype == AITER_DTYPE_i32 && sink->numel >= 1, "hbm_stream_read_cfg: sink must hold one int32");
        const int64_t bytes = (int64_t)src->numel * dtype_size(src->dtype);
        AA_CHECK(bytes % 16 == 0 && ((uintptr_t)src->ptr & 15) == 0,
                 "hbm_stream_read_cfg: src must be 16-byte aligned and a multiple of 16 bytes");
        AA_CHECK(grid > 0 && grid <= (1 << 20), "hbm_stream_read_cfg: grid out of range: ", grid);
        const CalibFn fn = pick_cfg(unroll, block, policy);
        AA_CHECK(fn, "hbm_stream_read_cfg: no kernel for unroll ", unroll, ", block ", block, ", policy ", policy,
                 " (unroll 1/2/4/8, block 64..1024, policy -1/0/1/2/3/16/17/18/19, or -2 with block 256: empty)");
        if (bytes == 0) return;
        fn(static_cast<const i32x4_t*>(src->ptr), bytes / 16, static_cast<int*>(sink->ptr), grid,
           reinterpret_cast<hipStream_t>(stream));
        AA_HIP(hipGetLastError());
    });
}

}  // extern "C"
