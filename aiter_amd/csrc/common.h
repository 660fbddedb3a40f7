// Shared definitions for the aiter_amd HIP library (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <sstream>
#include <stdexcept>
#include <string>

#include "aiter_amd.h"

namespace aiter_amd {

// ---------------------------------------------------------------------------
// Errors: every entry point runs its body through `safe_call`, which turns a
// C++ exception into status -1 plus a thread-local message (the contract of
// csrc/include/aiter_ctypes_error.h:83-147).
// ---------------------------------------------------------------------------
std::string& last_error();

template <typename... Args>
[[noreturn]] inline void fail(const char* fn, Args&&... args) {
    std::ostringstream os;
    os << fn << ": ";
    (os << ... << args);
    throw std::runtime_error(os.str());
}

#define AA_CHECK(cond, ...)                                     \
    do {                                                        \
        if (!(cond)) ::aiter_amd::fail(__func__, __VA_ARGS__);  \
    } while (0)

#define AA_HIP(call)                                                              \
    do {                                                                          \
        hipError_t e_ = (call);                                                   \
        if (e_ != hipSuccess)                                                     \
            ::aiter_amd::fail(__func__, #call, " -> ", hipGetErrorString(e_));    \
    } while (0)

template <typename F>
inline int safe_call(F&& f) {
    last_error().clear();
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        last_error() = e.what();
        return -1;
    } catch (...) {
        last_error() = "unknown C++ exception";
        return -1;
    }
}

inline size_t dtype_size(int dt) {
    switch (dt) {
        case AITER_DTYPE_fp8:
        case AITER_DTYPE_fp8_e8m0:
        case AITER_DTYPE_i4x2:
        case AITER_DTYPE_fp4x2:
        case AITER_DTYPE_i8:
        case AITER_DTYPE_u8: return 1;
        case AITER_DTYPE_fp16:
        case AITER_DTYPE_bf16:
        case AITER_DTYPE_i16: return 2;
        case AITER_DTYPE_fp32:
        case AITER_DTYPE_u32:
        case AITER_DTYPE_i32: return 4;
        case AITER_DTYPE_i64:
        case AITER_DTYPE_u64: return 8;
        default: return 0;
    }
}

inline const char* dtype_name(int dt) {
    static const char* names[] = {"fp8", "fp8_e8m0", "fp16", "bf16", "fp32", "i4x2", "fp4x2",
                                  "u32", "i32",      "i16",  "i8",   "u8",   "i64",  "u64"};
    return (dt >= 0 && dt < 14) ? names[dt] : "?";
}

inline bool is_byte_type(int dt) { return dtype_size(dt) == 1; }

inline void check_tensor(const aiter_tensor_t* t, const char* name, int ndim_min = 1) {
    if (!t) fail("check_tensor", name, " is NULL");
    if (t->ndim < ndim_min || t->ndim > 8) fail("check_tensor", name, " has ndim ", t->ndim);
    if (t->numel > 0 && !t->ptr) fail("check_tensor", name, " has a NULL data pointer");
}

// Row stride (elements) of a tensor viewed as [rows, cols] with unit inner
// stride; rejects layouts the kernels cannot address.
inline int64_t row_stride_2d(const aiter_tensor_t* t, const char* name) {
    if (t->strides[t->ndim - 1] != 1 && t->shape[t->ndim - 1] != 1)
        fail("row_stride_2d", name, " must have unit stride in the last dimension");
    if (t->ndim == 1) return t->shape[0];
    // collapse leading dims: they must be mutually contiguous
    for (int d = 0; d + 2 < t->ndim; ++d)
        if (t->shape[d] != 1 && t->strides[d] != t->strides[d + 1] * t->shape[d + 1])
            fail("row_stride_2d", name, " leading dimensions are not collapsible");
    return t->strides[t->ndim - 2];
}

inline int64_t rows_2d(const aiter_tensor_t* t) {
    int64_t r = 1;
    for (int d = 0; d + 1 < t->ndim; ++d) r *= t->shape[d];
    return r;
}

inline int64_t cols_2d(const aiter_tensor_t* t) { return t->shape[t->ndim - 1]; }

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (dev >= 0) {
            AA_HIP(hipGetDevice(&prev));
            if (prev != dev) AA_HIP(hipSetDevice(dev));
            else prev = -1;
        }
    }
    ~DeviceGuard() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

int device_cu_count(int dev);

// Library-owned device scratch of (device, stream), grown on demand (never
// inside graph capture: that raises); shared by the split-K GEMMs and the
// MoE sort, which are stream-ordered on one stream.
void* lib_workspace(int dev, hipStream_t st, size_t bytes);
// Zeroed int counters of (device, stream), grown on demand like the
// workspace; whoever uses them leaves them at zero when its launch ends.
int* lib_counters(int dev, hipStream_t st, size_t count);

}  // namespace aiter_amd

// ---------------------------------------------------------------------------
// Device-side helpers
// ---------------------------------------------------------------------------
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short i16x2_t __attribute__((ext_vector_type(2)));

#define AA_DEV __device__ __forceinline__

// f32 -> bf16 bits, round to nearest even (NaN kept quiet).
AA_DEV uint32_t f32_to_bf16_rne(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// two floats -> packed bf16 pair (v_cvt_pk_bf16_f32: round to nearest even)
AA_DEV uint32_t pack_bf16x2(float lo, float hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

AA_DEV float bf16_bits_to_f32(uint32_t b) { return __builtin_bit_cast(float, b << 16); }
