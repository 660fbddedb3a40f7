// HBM read-rate calibration: a plain streaming read with nothing else in the
// kernel, the attainable rate that the bandwidth-bound GEMMs (decode shapes)
// are compared against at the same byte count.  Not an operator: no
// counterpart in the reference.
#include "common.h"

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

}  // extern "C"
