// Shared host and device helpers of libkcr_hip.so: error reporting, tensor
// metadata checks and the 16-bit float element types.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <climits>
#include <cmath>
#include <type_traits>
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "../../include/kcr_hip.h"

namespace kcr {

// ---------------------------------------------------------------------------
// Errors: the entry points return a status and leave the message in a
// thread-local string, as the reference's exports return -1 after
// `Error::set_raised` (flash-attn2-rs/src/host/forward/mod.rs:828-831).
// ---------------------------------------------------------------------------
struct Error {
    int kind;
    std::string message;
};

void set_last_error(const std::string& message);

inline Error value_error(const std::string& m) { return Error{KCR_VALUE_ERROR, m}; }
inline Error type_error(const std::string& m) { return Error{KCR_TYPE_ERROR, m}; }
inline Error runtime_error(const std::string& m) { return Error{KCR_RUNTIME_ERROR, m}; }

// Runs `body` (which may throw kcr::Error) and converts the outcome to a status.
template <typename F>
int guarded(F&& body) {
    try {
        body();
        return KCR_OK;
    } catch (const Error& e) {
        set_last_error(e.message);
        return e.kind;
    } catch (const std::exception& e) {
        set_last_error(e.what());
        return KCR_RUNTIME_ERROR;
    }
}

inline void check_hip(hipError_t status, const char* what) {
    if (status != hipSuccess) {
        throw runtime_error(std::string(what) + ": " + hipGetErrorString(status));
    }
}

// Checks the launch that was just enqueued.
inline void check_launch(const char* what) { check_hip(hipGetLastError(), what); }

// Compute units of the current device, queried once per device.
inline int compute_units() {
    static std::atomic<int> cached[64] = {};
    int dev = 0;
    check_hip(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= 64) dev = 0;
    int cu = cached[dev].load(std::memory_order_relaxed);
    if (cu == 0) {
        check_hip(hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev),
                  "hipDeviceGetAttribute");
        if (cu <= 0) cu = 1;
        cached[dev].store(cu, std::memory_order_relaxed);
    }
    return cu;
}

// ---------------------------------------------------------------------------
// Tensor metadata.
// ---------------------------------------------------------------------------
inline int64_t numel(const kcr_tensor& t) {
    int64_t n = 1;
    for (int i = 0; i < t.ndim; ++i) n *= t.shape[i];
    return n;
}

inline bool is_contiguous(const kcr_tensor& t) {
    int64_t expected = 1;
    for (int i = t.ndim - 1; i >= 0; --i) {
        if (t.shape[i] != 1 && t.strides[i] != expected) return false;
        expected *= t.shape[i];
    }
    return true;
}

inline size_t element_size(int dtype) {
    switch (dtype) {
        case KCR_FLOAT32: return 4;
        case KCR_FLOAT16: return 2;
        case KCR_BFLOAT16: return 2;
        case KCR_INT32: return 4;
        case KCR_INT64: return 8;
        case KCR_FLOAT64: return 8;
        default: return 0;
    }
}

std::string shape_string(const kcr_tensor& t);
std::string shape_string(const std::vector<int64_t>& shape);
std::vector<int64_t> shape_of(const kcr_tensor& t);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---------------------------------------------------------------------------
// Device element types. Arithmetic is done in f32; bf16/f16 are storage types,
// rounded to nearest even when narrowed.
// ---------------------------------------------------------------------------
struct bf16_t {
    uint16_t bits;
};
struct f16_t {
    uint16_t bits;
};

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits) {
    return __uint_as_float(bits << 16);
}

// Round-to-nearest-even f32 -> bf16 bits; NaN stays a quiet NaN.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) | 0x40u) & 0xffffu;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

// Two f32 -> packed bf16x2 (lo in the low half), round to nearest even.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits) {
    _Float16 h = __builtin_bit_cast(_Float16, static_cast<uint16_t>(bits));
    return static_cast<float>(h);
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
    _Float16 h = static_cast<_Float16>(f);
    return __builtin_bit_cast(uint16_t, h);
}

template <typename T>
struct Elem;

template <>
struct Elem<float> {
    using storage = float;
    static __device__ __forceinline__ float load(const float* p) { return *p; }
    static __device__ __forceinline__ void store(float* p, float v) { *p = v; }
    static __device__ __forceinline__ float round(float v) { return v; }
};

template <>
struct Elem<bf16_t> {
    using storage = uint16_t;
    static __device__ __forceinline__ float to_f32(uint32_t bits) { return bf16_bits_to_f32(bits); }
    // Round to nearest even (v_cvt_pk_bf16_f32).
    static __device__ __forceinline__ uint32_t from_f32(float v) {
        return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
    }
    static __device__ __forceinline__ float load(const bf16_t* p) { return to_f32(p->bits); }
    static __device__ __forceinline__ void store(bf16_t* p, float v) {
        p->bits = static_cast<uint16_t>(from_f32(v));
    }
    static __device__ __forceinline__ float round(float v) { return to_f32(from_f32(v)); }
};

template <>
struct Elem<f16_t> {
    using storage = uint16_t;
    static __device__ __forceinline__ float to_f32(uint32_t bits) { return f16_bits_to_f32(bits); }
    static __device__ __forceinline__ uint32_t from_f32(float v) { return f32_to_f16_bits(v); }
    static __device__ __forceinline__ float load(const f16_t* p) { return to_f32(p->bits); }
    static __device__ __forceinline__ void store(f16_t* p, float v) {
        p->bits = static_cast<uint16_t>(from_f32(v));
    }
    static __device__ __forceinline__ float round(float v) { return to_f32(from_f32(v)); }
};

// A value the compiler must materialise as an f32 before its next use. An
// f32 result narrowed to f16 is otherwise folded into one mixed-precision
// instruction (v_fma_mixlo_f16) that rounds the exact result to f16 once,
// where an f32 computation rounds to f32 first and then to f16 (the two differ
// at f16 ties of the f32 value). Used where results must match that order.
__device__ __forceinline__ float as_f32(float v) {
    asm("" : "+v"(v));
    return v;
}

// 16-byte vectors of 8 x 16-bit or 4 x 32-bit elements.
using u32x4 = __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t;

// Eight elements widened to f32, from one 16-byte word (element 2i is the low
// half of word i).
template <typename T>
__device__ __forceinline__ void unpack8(const u32x4& w, float (&f)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = Elem<T>::to_f32(w[i] & 0xffffu);
        f[2 * i + 1] = Elem<T>::to_f32(w[i] >> 16);
    }
}

// Two f32 -> one word of two 16-bit elements (lo in the low half), round to
// nearest even: a single v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32 on gfx950.
template <typename T>
__device__ __forceinline__ uint32_t pack_pair(float lo, float hi) {
    using f32x2 = float __attribute__((ext_vector_type(2)));
    const f32x2 v = {lo, hi};
    if constexpr (std::is_same<T, bf16_t>::value) {
        using bf16x2 = __bf16 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
    } else {
        using f16x2 = _Float16 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
    }
}

template <typename T>
__device__ __forceinline__ u32x4 pack8(const float (&f)[8]) {
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = pack_pair<T>(f[2 * i], f[2 * i + 1]);
    return w;
}

// Wave64 sum: every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) v = fmaxf(v, __shfl_xor(v, offset, 64));
    return v;
}

}  // namespace kcr

namespace kcr {
// Host tensors reach the C ABI with device == -1 (e.g. when a caller only wants
// the argument validation); the kernels run on GPU memory only.
inline void require_device(const kcr_tensor* t, const char* name) {
    if (t && t->device < 0) {
        throw value_error(std::string(name) + " must be a GPU tensor");
    }
}
}  // namespace kcr
