// Gated and element-wise activations (activation-rs).
//
// Reference: activation-rs/src/device.rs:18-80 (kernels), activation-rs/src/ops.rs:27-265
// (validation and exports), activation-rs/src/activation.rs:34-122 (element math).
//
// MI355X design: the ops are pure streaming kernels (HBM-bound). Instead of the
// reference's one-block-per-token scalar loop, every thread moves 16-byte vectors
// (8 x bf16/f16 or 4 x f32) of the gate and up halves and writes one 16-byte
// vector of output; a thread keeps UNROLL independent vectors in flight so each
// wave has enough outstanding loads to cover HBM latency. The flat vector index
// space (rows x vectors-per-row) is walked with a grid-stride loop. Rows whose
// width or base address does not allow 16-byte access take a scalar kernel.
//
// Rounding follows the reference exactly: the activation is evaluated in f32 and
// rounded to the element type, then the product is formed in f32 and rounded
// again (activation.rs:42-46, element.rs:103-106). The element-wise GELU
// variants round at every step where the reference does (activation.rs:79-104).
//
// 16-bit element types: an activation of a bf16 / f16 input has only 65536
// possible arguments, so each one is a 128 KB table of result bits, built once
// per device with the reference's expression and correctly rounded f32 values
// of exp / erf / tanh (evaluated in f64). The streaming kernels copy the table
// into LDS (gfx950 has 160 KB per CU, so one 1024-thread block per CU holds it)
// and replace the transcendental arithmetic by one LDS read per element. The
// results are the table's, bit for bit, whichever kernel runs; the product with
// the other half is exact in f32 and rounded once, as in the reference.
#include "common.h"

#include <algorithm>
#include <mutex>
#include <vector>

namespace kcr {

enum Act : int {
    ACT_SILU = 0,
    ACT_GELU = 1,
    ACT_GELU_TANH = 2,
    ACT_GELU_NEW = 3,
    ACT_GELU_FAST = 4,
    ACT_GELU_QUICK = 5,
    ACT_FATRELU = 6,
};

// f32 -> T -> f32, from the rounded f32 value (the reference's order).
template <typename T>
__device__ __forceinline__ float rnd(float v) {
    return Elem<T>::round(as_f32(v));
}

// The f32 expression of activation A (activation.rs:42-122) with the device
// libm; used for f32 elements (16-bit elements read tables, below).
template <typename T, int A>
__device__ __forceinline__ float apply_act(float f, float threshold) {
    if constexpr (A == ACT_SILU) {
        // activation.rs:42-46: f / (1 + exp(-f))
        return rnd<T>(f / (1.0f + expf(-f)));
    } else if constexpr (A == ACT_GELU) {
        // activation.rs:53-58: f * 0.5 * (1 + erf(f / sqrt(2)))
        const float alpha = 0.70710678118654752440f;
        return rnd<T>(f * 0.5f * (1.0f + erff(f * alpha)));
    } else if constexpr (A == ACT_GELU_TANH) {
        // activation.rs:64-76: beta = sqrt(2) * 2/sqrt(pi) * 0.5 (f64 -> f32),
        // inner = beta * fma(kappa, f^3, f)
        const float beta = static_cast<float>(1.4142135623730951 * 1.1283791670955126 * 0.5);
        const float kappa = 0.044715f;
        const float x_cube = f * f * f;
        const float inner = beta * __builtin_fmaf(kappa, x_cube, f);
        return rnd<T>(0.5f * f * (1.0f + tanhf(inner)));
    } else if constexpr (A == ACT_GELU_NEW) {
        // activation.rs:79-90, every intermediate in T.
        const float x3 = rnd<T>(rnd<T>(f * f) * f);
        const float inner = rnd<T>(f + rnd<T>(0.044715f * x3));
        const float t = rnd<T>(tanhf(rnd<T>(0.79788456f * inner)));
        return rnd<T>(rnd<T>(rnd<T>(0.5f) * f) * rnd<T>(rnd<T>(1.0f) + t));
    } else if constexpr (A == ACT_GELU_FAST) {
        // activation.rs:92-104
        const float scaled = rnd<T>(f * 0.79788456f);
        const float cubic = rnd<T>(rnd<T>(1.0f) + rnd<T>(rnd<T>(0.044715f * f) * f));
        const float t = rnd<T>(tanhf(rnd<T>(scaled * cubic)));
        return rnd<T>(rnd<T>(rnd<T>(0.5f) * f) * rnd<T>(rnd<T>(1.0f) + t));
    } else if constexpr (A == ACT_GELU_QUICK) {
        // activation.rs:106-115
        return rnd<T>(f / (1.0f + expf(-1.702f * f)));
    } else {
        // activation.rs:117-122 (FATReLU)
        return rnd<T>(f > threshold ? f : 0.0f);
    }
}

// ---------------------------------------------------------------------------
// Exact activations of 16-bit inputs, and their tables.
// ---------------------------------------------------------------------------

// Correctly rounded f32 values of the elementary functions: the f64 result
// (accurate to about one f64 ulp) rounded once to f32.
__device__ __forceinline__ float exp_cr(float x) { return static_cast<float>(exp(static_cast<double>(x))); }
__device__ __forceinline__ float erf_cr(float x) { return static_cast<float>(erf(static_cast<double>(x))); }
__device__ __forceinline__ float tanh_cr(float x) { return static_cast<float>(tanh(static_cast<double>(x))); }
// IEEE f32 quotient: the f64 quotient of two floats rounds to the same float.
__device__ __forceinline__ float div_rn(float a, float b) {
    return static_cast<float>(static_cast<double>(a) / static_cast<double>(b));
}

// The reference's expression for A (activation.rs:42-115) with every f32
// operation rounded separately (no contraction) and the elementary functions
// correctly rounded; returns the result rounded to T.
template <typename T, int A>
__device__ float act_exact(float f) {
#pragma clang fp contract(off)
    if constexpr (A == ACT_SILU) {
        return rnd<T>(div_rn(f, 1.0f + exp_cr(-f)));
    } else if constexpr (A == ACT_GELU) {
        const float alpha = 0.70710678118654752440f;
        return rnd<T>(f * 0.5f * (1.0f + erf_cr(f * alpha)));
    } else if constexpr (A == ACT_GELU_TANH) {
        const float beta = static_cast<float>(1.4142135623730951 * 1.1283791670955126 * 0.5);
        const float kappa = 0.044715f;
        const float x_cube = f * f * f;
        const float inner = beta * __builtin_fmaf(kappa, x_cube, f);
        return rnd<T>(0.5f * f * (1.0f + tanh_cr(inner)));
    } else if constexpr (A == ACT_GELU_NEW) {
        const float x3 = rnd<T>(rnd<T>(f * f) * f);
        const float inner = rnd<T>(f + rnd<T>(0.044715f * x3));
        const float t = rnd<T>(tanh_cr(rnd<T>(0.79788456f * inner)));
        return rnd<T>(rnd<T>(rnd<T>(0.5f) * f) * rnd<T>(rnd<T>(1.0f) + t));
    } else if constexpr (A == ACT_GELU_FAST) {
        const float scaled = rnd<T>(f * 0.79788456f);
        const float cubic = rnd<T>(rnd<T>(1.0f) + rnd<T>(rnd<T>(0.044715f * f) * f));
        const float t = rnd<T>(tanh_cr(rnd<T>(scaled * cubic)));
        return rnd<T>(rnd<T>(rnd<T>(0.5f) * f) * rnd<T>(rnd<T>(1.0f) + t));
    } else {
        static_assert(A == ACT_GELU_QUICK, "activations with a table");
        return rnd<T>(div_rn(f, 1.0f + exp_cr(-1.702f * f)));
    }
}

// Table slots: [dtype (0 bf16, 1 f16)][activation], 65536 result bits each.
constexpr int kLutActs = 6;  // ACT_SILU .. ACT_GELU_QUICK
template <int A>
constexpr bool has_lut() {
    return A >= ACT_SILU && A <= ACT_GELU_QUICK;
}
template <typename T>
constexpr int lut_dtype() {
    return std::is_same<T, bf16_t>::value ? 0 : 1;
}
template <typename T, int A>
constexpr int lut_slot() {
    return lut_dtype<T>() * kLutActs + A;
}

// 12 x 128 KB in device memory, filled by build_act_luts once per device.
__device__ uint16_t g_act_lut[2 * kLutActs][65536];

template <typename T>
__device__ void fill_lut_entry(int act, uint32_t bits) {
    const float f = Elem<T>::to_f32(bits);
    uint32_t r;
    switch (act) {
        case ACT_SILU: r = Elem<T>::from_f32(act_exact<T, ACT_SILU>(f)); break;
        case ACT_GELU: r = Elem<T>::from_f32(act_exact<T, ACT_GELU>(f)); break;
        case ACT_GELU_TANH: r = Elem<T>::from_f32(act_exact<T, ACT_GELU_TANH>(f)); break;
        case ACT_GELU_NEW: r = Elem<T>::from_f32(act_exact<T, ACT_GELU_NEW>(f)); break;
        case ACT_GELU_FAST: r = Elem<T>::from_f32(act_exact<T, ACT_GELU_FAST>(f)); break;
        default: r = Elem<T>::from_f32(act_exact<T, ACT_GELU_QUICK>(f)); break;
    }
    g_act_lut[lut_dtype<T>() * kLutActs + act][bits] = static_cast<uint16_t>(r);
}

// One thread per (table, input): grid 2 * kLutActs * 256 blocks of 256.
__global__ void __launch_bounds__(256) build_act_luts() {
    const uint32_t id = blockIdx.x * 256u + threadIdx.x;
    const int slot = static_cast<int>(id >> 16);
    const uint32_t bits = id & 0xffffu;
    if (slot < kLutActs) {
        fill_lut_entry<bf16_t>(slot, bits);
    } else if (slot < 2 * kLutActs) {
        fill_lut_entry<f16_t>(slot - kLutActs, bits);
    }
}

// Result bits of activation A at 16-bit input bits, from the global table
// (the scalar kernels; the streaming kernels read their LDS copy).
template <typename T, int A>
__device__ __forceinline__ float act_lut_global(uint32_t bits) {
    return Elem<T>::to_f32(g_act_lut[lut_slot<T, A>()][bits]);
}

// act(f) rounded to T: the table for 16-bit T, else the f32 expression.
template <typename T, int A>
__device__ __forceinline__ float act_value(float f, float threshold) {
    if constexpr (sizeof(typename Elem<T>::storage) == 2 && has_lut<A>()) {
        return act_lut_global<T, A>(Elem<T>::from_f32(f));
    } else {
        return apply_act<T, A>(f, threshold);
    }
}

template <typename T, int A, bool ACT_FIRST>
__device__ __forceinline__ float gated(float x, float y, float threshold) {
    if constexpr (ACT_FIRST) {
        return act_value<T, A>(x, threshold) * y;
    } else {
        return x * act_value<T, A>(y, threshold);
    }
}

// Elements per 16-byte vector.
template <typename T>
constexpr int vec_elems() {
    return 16 / sizeof(typename Elem<T>::storage);
}

template <typename T>
__device__ __forceinline__ void widen(const u32x4& w, float (&f)[16 / sizeof(typename Elem<T>::storage)]) {
    if constexpr (sizeof(typename Elem<T>::storage) == 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) f[i] = __uint_as_float(w[i]);
    } else {
        unpack8<T>(w, f);
    }
}

template <typename T>
__device__ __forceinline__ u32x4 narrow(const float (&f)[16 / sizeof(typename Elem<T>::storage)]) {
    if constexpr (sizeof(typename Elem<T>::storage) == 4) {
        u32x4 w;
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = __float_as_uint(f[i]);
        return w;
    } else {
        return pack8<T>(f);
    }
}

constexpr int kThreads = 256;
// Two 16-byte vectors per thread and one thread per pair: measured on MI355X,
// a one-shot grid with non-temporal accesses streams best (a grid-stride loop
// over fewer blocks reached ~4.1 TB/s, this shape ~6.3 TB/s).
constexpr int kUnroll = 2;

// Gated kernel: kGatedUnroll consecutive 256-vector chunks per block and
// iteration, over a grid capped at kGatedBlocks (grid-stride). Measured on
// MI355X at the gated ops' 2:1 read:write mix: +0.7 % over the one-shot shape
// (6.32 vs 6.28 TB/s); 8192 blocks lose 4 %.
constexpr int kGatedUnroll = 4;
constexpr uint64_t kGatedBlocks = 32768;

// Gated activation over 16-byte vectors. `vpr` = vectors per output row
// (d / VEC); `total` = rows * vpr. Input rows are 2 * vpr vectors wide.
template <typename T, int A, bool ACT_FIRST, bool WIDE>
__global__ void __launch_bounds__(kThreads) act_and_mul_vec(u32x4* __restrict__ out,
                                                            const u32x4* __restrict__ in,
                                                            uint64_t total, uint32_t vpr,
                                                            float threshold) {
    constexpr int VEC = vec_elems<T>();
    // Each block takes kGatedUnroll consecutive 256-vector chunks per iteration and
    // strides over the grid (a capped grid keeps kGatedUnroll x 2 loads in flight per
    // lane on every wave).
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads * kGatedUnroll;
    uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads * kGatedUnroll + threadIdx.x;
    for (; i < total; i += stride) {
        u32x4 xs[kGatedUnroll], ys[kGatedUnroll];
        uint64_t oidx[kGatedUnroll];
        bool ok[kGatedUnroll];
#pragma unroll
        for (int u = 0; u < kGatedUnroll; ++u) {
            const uint64_t j = i + static_cast<uint64_t>(u) * kThreads;
            ok[u] = j < total;
            uint64_t row, col;
            if constexpr (WIDE) {
                row = j / vpr;
                col = j - row * vpr;
            } else {
                const uint32_t j32 = static_cast<uint32_t>(j);
                row = j32 / vpr;
                col = j32 - static_cast<uint32_t>(row) * vpr;
            }
            oidx[u] = j;
            const uint64_t base = row * 2 * vpr + col;
            if (ok[u]) {
                xs[u] = __builtin_nontemporal_load(in + base);
                ys[u] = __builtin_nontemporal_load(in + base + vpr);
            }
        }
#pragma unroll
        for (int u = 0; u < kGatedUnroll; ++u) {
            if (!ok[u]) continue;
            float x[VEC], y[VEC], r[VEC];
            widen<T>(xs[u], x);
            widen<T>(ys[u], y);
#pragma unroll
            for (int e = 0; e < VEC; ++e) r[e] = gated<T, A, ACT_FIRST>(x[e], y[e], threshold);
            __builtin_nontemporal_store(narrow<T>(r), out + oidx[u]);
        }
    }
}

// Scalar fallback for widths that are not a multiple of the vector or for
// misaligned storage: one element per thread, grid-stride.
template <typename T, int A, bool ACT_FIRST>
__global__ void __launch_bounds__(kThreads) act_and_mul_scalar(T* __restrict__ out,
                                                               const T* __restrict__ in,
                                                               uint64_t total, uint64_t d,
                                                               float threshold) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < total;
         i += stride) {
        const uint64_t row = i / d;
        const uint64_t col = i - row * d;
        const float x = Elem<T>::load(in + row * 2 * d + col);
        const float y = Elem<T>::load(in + row * 2 * d + d + col);
        Elem<T>::store(out + i, ACT_FIRST ? act_value<T, A>(x, threshold) * y
                                          : x * act_value<T, A>(y, threshold));
    }
}

template <typename T, int A>
__global__ void __launch_bounds__(kThreads) activation_vec(u32x4* __restrict__ out,
                                                           const u32x4* __restrict__ in,
                                                           uint64_t total) {
    constexpr int VEC = vec_elems<T>();
    // Same memory shape as act_and_mul_vec: kGatedUnroll consecutive 256-vector
    // chunks per block and iteration over a capped, grid-strided grid.
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads * kGatedUnroll;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads * kGatedUnroll + threadIdx.x; i < total;
         i += stride) {
        u32x4 xs[kGatedUnroll];
#pragma unroll
        for (int u = 0; u < kGatedUnroll; ++u) {
            const uint64_t j = i + static_cast<uint64_t>(u) * kThreads;
            if (j < total) xs[u] = __builtin_nontemporal_load(in + j);
        }
#pragma unroll
        for (int u = 0; u < kGatedUnroll; ++u) {
            const uint64_t j = i + static_cast<uint64_t>(u) * kThreads;
            if (j >= total) continue;
            float x[VEC], r[VEC];
            widen<T>(xs[u], x);
#pragma unroll
            for (int e = 0; e < VEC; ++e) r[e] = act_value<T, A>(x[e], 0.0f);
            __builtin_nontemporal_store(narrow<T>(r), out + j);
        }
    }
}

// Streaming kernels over a table in LDS. A block is 1024 threads (the 128 KB
// table leaves no room for a second block on the CU), each thread U 16-byte
// vectors of each input per iteration. Measured on MI355X (silu_and_mul,
// 16384 x 28672 bf16): a grid that covers the input in one pass (every block
// one iteration, blocks dispatched as CUs free up) streams at 6.35-6.39 TB/s;
// capping the grid at 1, 4 or 16 blocks per CU and looping gave 5.54, 5.79
// and 6.06 TB/s, and 8 vectors per thread (half the blocks, one pass) 6.0:
// the dispatcher's dynamic balance across CUs is worth more than the 128 KB
// table copy each block makes from L2. The element-wise
// kernels (one input) run best with U = 2 and at most 24 blocks per CU
// (6.12 TB/s against 5.65 for one pass at U = 4).
constexpr int kLutThreads = 1024;
constexpr int kGatedLutUnroll = 4;
constexpr int kEltLutUnroll = 2;
constexpr int kEltLutBlocksPerCu = 24;

// Copies table `slot` into `lut` (128 KB of LDS) and waits for the block.
__device__ __forceinline__ void load_lut(uint16_t* lut, int slot) {
    const u32x4* src = reinterpret_cast<const u32x4*>(g_act_lut[slot]);
    u32x4* dst = reinterpret_cast<u32x4*>(lut);
#pragma unroll
    for (int i = 0; i < 65536 * 2 / 16 / kLutThreads; ++i) dst[threadIdx.x + i * kLutThreads] = src[threadIdx.x + i * kLutThreads];
    __syncthreads();
}

template <typename T, int A, bool ACT_FIRST, bool WIDE>
__global__ void __launch_bounds__(kLutThreads) act_and_mul_lut(u32x4* __restrict__ out,
                                                               const u32x4* __restrict__ in,
                                                               uint64_t total, uint32_t vpr) {
    constexpr int U = kGatedLutUnroll;
    __shared__ uint16_t lut[65536];
    load_lut(lut, lut_slot<T, A>());
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kLutThreads * U;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kLutThreads * U + threadIdx.x; i < total;
         i += stride) {
        u32x4 xs[U], ys[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint64_t j = i + static_cast<uint64_t>(u) * kLutThreads;
            uint64_t row, col;
            if constexpr (WIDE) {
                row = j / vpr;
                col = j - row * vpr;
            } else {
                const uint32_t j32 = static_cast<uint32_t>(j);
                row = j32 / vpr;
                col = j32 - static_cast<uint32_t>(row) * vpr;
            }
            const uint64_t base = row * 2 * vpr + col;
            if (j < total) {
                xs[u] = __builtin_nontemporal_load(in + base);
                ys[u] = __builtin_nontemporal_load(in + base + vpr);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint64_t j = i + static_cast<uint64_t>(u) * kLutThreads;
            if (j >= total) continue;
            u32x4 r;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                // a: the half the activation applies to; b: the other half.
                const uint32_t a = ACT_FIRST ? xs[u][k] : ys[u][k];
                const uint32_t b = ACT_FIRST ? ys[u][k] : xs[u][k];
                const float al = Elem<T>::to_f32(lut[a & 0xffffu]);
                const float ah = Elem<T>::to_f32(lut[a >> 16]);
                // Products of two 16-bit values are exact in f32: one rounding.
                r[k] = pack_pair<T>(al * Elem<T>::to_f32(b & 0xffffu), ah * Elem<T>::to_f32(b >> 16));
            }
            __builtin_nontemporal_store(r, out + j);
        }
    }
}

// Element-wise: out = table[in], no arithmetic at all.
template <typename T, int A>
__global__ void __launch_bounds__(kLutThreads) activation_lut(u32x4* __restrict__ out,
                                                              const u32x4* __restrict__ in,
                                                              uint64_t total) {
    constexpr int U = kEltLutUnroll;
    __shared__ uint16_t lut[65536];
    load_lut(lut, lut_slot<T, A>());
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kLutThreads * U;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kLutThreads * U + threadIdx.x; i < total;
         i += stride) {
        u32x4 xs[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint64_t j = i + static_cast<uint64_t>(u) * kLutThreads;
            if (j < total) xs[u] = __builtin_nontemporal_load(in + j);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint64_t j = i + static_cast<uint64_t>(u) * kLutThreads;
            if (j >= total) continue;
            u32x4 r;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                r[k] = static_cast<uint32_t>(lut[xs[u][k] & 0xffffu]) |
                       (static_cast<uint32_t>(lut[xs[u][k] >> 16]) << 16);
            __builtin_nontemporal_store(r, out + j);
        }
    }
}

template <typename T, int A>
__global__ void __launch_bounds__(kThreads) activation_scalar(T* __restrict__ out,
                                                              const T* __restrict__ in,
                                                              uint64_t total) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < total;
         i += stride) {
        Elem<T>::store(out + i, act_value<T, A>(Elem<T>::load(in + i), 0.0f));
    }
}

namespace {

// One block per kThreads * kUnroll items (the kernels still loop, so any cap
// stays correct); capped at the grid-x limit.
unsigned grid_for(uint64_t work_items) {
    const uint64_t per_block = static_cast<uint64_t>(kThreads) * kUnroll;
    uint64_t blocks = (work_items + per_block - 1) / per_block;
    const uint64_t cap = 2147483647ull;
    if (blocks > cap) blocks = cap;
    if (blocks == 0) blocks = 1;
    return static_cast<unsigned>(blocks);
}

// Builds the activation tables of the current device on its first use (one
// kernel on a private stream, waited for, so the tables are complete before
// any stream of the caller reads them). Later calls return at once.
void ensure_luts() {
    static std::mutex mu;
    static std::vector<char> built;
    int device = 0;
    check_hip(hipGetDevice(&device), "hipGetDevice");
    std::lock_guard<std::mutex> lock(mu);
    if (static_cast<size_t>(device) < built.size() && built[device]) return;
    hipStream_t s;
    check_hip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
    build_act_luts<<<2 * kLutActs * 256, 256, 0, s>>>();
    const hipError_t launched = hipGetLastError();
    const hipError_t done = hipStreamSynchronize(s);
    hipStreamDestroy(s);
    check_hip(launched, "launch build_act_luts");
    check_hip(done, "build_act_luts");
    if (built.size() <= static_cast<size_t>(device)) built.resize(device + 1, 0);
    built[device] = 1;
}

// Grid of a table kernel: enough blocks of kLutThreads x unroll vectors to
// cover the input once, at most `cap`.
unsigned lut_grid(uint64_t total_vectors, int unroll, uint64_t cap) {
    const uint64_t per_block = static_cast<uint64_t>(kLutThreads) * unroll;
    const uint64_t need = (total_vectors + per_block - 1) / per_block;
    return static_cast<unsigned>(std::max<uint64_t>(1, std::min<uint64_t>(need, cap)));
}

struct Launch {
    int64_t tokens = 0;
    int64_t d = 0;
    bool empty = false;
};

// Validation of activation-rs/src/ops.rs:27-78 (launch_config) plus the
// dtype and contiguity checks of ops.rs:173-189 and kernels_cuda's view.
Launch validate(const kcr_tensor* out, const kcr_tensor* input, bool gated) {
    if (!out || !input) throw value_error("out and input are required");
    if (input->ndim == 0) throw value_error("input must have at least one dimension");
    const int64_t last = input->shape[input->ndim - 1];
    if (gated && last % 2 != 0) {
        throw value_error("the last dimension of input must be even, got " + std::to_string(last));
    }
    const int64_t d = gated ? last / 2 : last;
    std::vector<int64_t> expected(input->shape, input->shape + input->ndim - 1);
    expected.push_back(d);
    if (shape_of(*out) != expected) {
        throw value_error("out must have shape " + shape_string(expected) + ", got " +
                          shape_string(*out));
    }
    if (input->dtype != out->dtype) throw value_error("input and out must have the same dtype");
    int64_t tokens = 1;
    for (int i = 0; i + 1 < input->ndim; ++i) tokens *= input->shape[i];
    Launch l;
    l.tokens = tokens;
    l.d = d;
    if (tokens == 0 || d == 0) {
        l.empty = true;
        return l;
    }
    const int64_t max_grid_x = 2147483647;
    if (tokens > max_grid_x) {
        throw value_error("input has " + std::to_string(tokens) + " rows, at most " +
                          std::to_string(max_grid_x) + " are supported");
    }
    if (d > 4294967295ll) {
        throw value_error("rows of " + std::to_string(d) + " elements are not supported");
    }
    if (input->dtype != KCR_FLOAT16 && input->dtype != KCR_BFLOAT16 &&
        input->dtype != KCR_FLOAT32) {
        throw value_error("unsupported dtype, expected float16, bfloat16 or float32");
    }
    if (!is_contiguous(*input)) throw value_error("input must be contiguous");
    if (!is_contiguous(*out)) throw value_error("out must be contiguous");
    require_device(input, "input");
    require_device(out, "out");
    return l;
}

template <typename T, int A, bool ACT_FIRST>
void launch_gated_t(const kcr_tensor* out, const kcr_tensor* input, const Launch& l,
                    float threshold, hipStream_t stream) {
    constexpr int VEC = vec_elems<T>();
    const uint64_t total_elems = static_cast<uint64_t>(l.tokens) * static_cast<uint64_t>(l.d);
    const bool vec = (l.d % VEC == 0) && aligned16(out->data) && aligned16(input->data);
    if (vec) {
        const uint64_t vpr = static_cast<uint64_t>(l.d) / VEC;
        const uint64_t total = static_cast<uint64_t>(l.tokens) * vpr;
        if constexpr (sizeof(typename Elem<T>::storage) == 2 && has_lut<A>()) {
            ensure_luts();
            const unsigned grid = lut_grid(total, kGatedLutUnroll, 2147483647ull);
            // 32-bit index math when every flat index, plus one grid stride of
            // unrolled look-ahead, stays below 2^32.
            const uint64_t reach = total + static_cast<uint64_t>(grid) * kLutThreads * kGatedLutUnroll;
            if (reach < (1ull << 32)) {
                act_and_mul_lut<T, A, ACT_FIRST, false><<<grid, kLutThreads, 0, stream>>>(
                    static_cast<u32x4*>(out->data), static_cast<const u32x4*>(input->data), total,
                    static_cast<uint32_t>(vpr));
            } else {
                act_and_mul_lut<T, A, ACT_FIRST, true><<<grid, kLutThreads, 0, stream>>>(
                    static_cast<u32x4*>(out->data), static_cast<const u32x4*>(input->data), total,
                    static_cast<uint32_t>(vpr));
            }
            check_launch("launch act_and_mul");
            return;
        }
        const uint64_t need = (total + kThreads * kGatedUnroll - 1) / (kThreads * kGatedUnroll);
        const unsigned grid = static_cast<unsigned>(std::max<uint64_t>(1, std::min<uint64_t>(need, kGatedBlocks)));
        // 32-bit index math when every flat index, plus one grid stride of
        // unrolled look-ahead, stays below 2^32.
        const uint64_t reach = total + static_cast<uint64_t>(grid) * kThreads * kGatedUnroll;
        if (reach < (1ull << 32)) {
            act_and_mul_vec<T, A, ACT_FIRST, false><<<grid, kThreads, 0, stream>>>(
                static_cast<u32x4*>(out->data), static_cast<const u32x4*>(input->data), total,
                static_cast<uint32_t>(vpr), threshold);
        } else {
            act_and_mul_vec<T, A, ACT_FIRST, true><<<grid, kThreads, 0, stream>>>(
                static_cast<u32x4*>(out->data), static_cast<const u32x4*>(input->data), total,
                static_cast<uint32_t>(vpr), threshold);
        }
    } else {
        if constexpr (sizeof(typename Elem<T>::storage) == 2 && has_lut<A>()) ensure_luts();
        const unsigned grid = grid_for(total_elems);
        act_and_mul_scalar<T, A, ACT_FIRST><<<grid, kThreads, 0, stream>>>(
            static_cast<T*>(out->data), static_cast<const T*>(input->data), total_elems,
            static_cast<uint64_t>(l.d), threshold);
    }
    check_launch("launch act_and_mul");
}

template <int A, bool ACT_FIRST>
int run_gated(const kcr_tensor* out, const kcr_tensor* input, double threshold, void* stream) {
    return guarded([&] {
        const Launch l = validate(out, input, true);
        if (l.empty) return;
        auto s = static_cast<hipStream_t>(stream);
        const float thr = static_cast<float>(threshold);
        switch (input->dtype) {
            case KCR_FLOAT16: launch_gated_t<f16_t, A, ACT_FIRST>(out, input, l, thr, s); break;
            case KCR_BFLOAT16: launch_gated_t<bf16_t, A, ACT_FIRST>(out, input, l, thr, s); break;
            default: launch_gated_t<float, A, ACT_FIRST>(out, input, l, thr, s); break;
        }
    });
}

template <typename T, int A>
void launch_elementwise_t(const kcr_tensor* out, const kcr_tensor* input, const Launch& l,
                          hipStream_t stream) {
    constexpr int VEC = vec_elems<T>();
    const uint64_t total_elems = static_cast<uint64_t>(l.tokens) * static_cast<uint64_t>(l.d);
    constexpr bool kTable = sizeof(typename Elem<T>::storage) == 2 && has_lut<A>();
    if constexpr (kTable) ensure_luts();
    if (total_elems % VEC == 0 && aligned16(out->data) && aligned16(input->data)) {
        const uint64_t total = total_elems / VEC;
        if constexpr (kTable) {
            const unsigned grid = lut_grid(total, kEltLutUnroll,
                                           static_cast<uint64_t>(kEltLutBlocksPerCu) * compute_units());
            activation_lut<T, A><<<grid, kLutThreads, 0, stream>>>(
                static_cast<u32x4*>(out->data), static_cast<const u32x4*>(input->data), total);
            check_launch("launch activation");
            return;
        }
        const uint64_t need = (total + kThreads * kGatedUnroll - 1) / (kThreads * kGatedUnroll);
        const unsigned grid = static_cast<unsigned>(std::max<uint64_t>(1, std::min(need, kGatedBlocks)));
        activation_vec<T, A><<<grid, kThreads, 0, stream>>>(
            static_cast<u32x4*>(out->data), static_cast<const u32x4*>(input->data), total);
    } else {
        activation_scalar<T, A><<<grid_for(total_elems), kThreads, 0, stream>>>(
            static_cast<T*>(out->data), static_cast<const T*>(input->data), total_elems);
    }
    check_launch("launch activation");
}

template <int A>
int run_elementwise(const kcr_tensor* out, const kcr_tensor* input, void* stream) {
    return guarded([&] {
        const Launch l = validate(out, input, false);
        if (l.empty) return;
        auto s = static_cast<hipStream_t>(stream);
        switch (input->dtype) {
            case KCR_FLOAT16: launch_elementwise_t<f16_t, A>(out, input, l, s); break;
            case KCR_BFLOAT16: launch_elementwise_t<bf16_t, A>(out, input, l, s); break;
            default: launch_elementwise_t<float, A>(out, input, l, s); break;
        }
    });
}

}  // namespace
}  // namespace kcr

using namespace kcr;

extern "C" {

int kcr_silu_and_mul(const kcr_tensor* out, const kcr_tensor* input, void* stream) {
    return run_gated<ACT_SILU, true>(out, input, 0.0, stream);
}
int kcr_mul_and_silu(const kcr_tensor* out, const kcr_tensor* input, void* stream) {
    return run_gated<ACT_SILU, false>(out, input, 0.0, stream);
}
int kcr_gelu_and_mul(const kcr_tensor* out, const kcr_tensor* input, void* stream) {
    return run_gated<ACT_GELU, true>(out, input, 0.0, stream);
}
int kcr_gelu_tanh_and_mul(const kcr_tensor* out, const kcr_tensor* input, void* stream) {
    return run_gated<ACT_GELU_TANH, true>(out, input, 0.0, stream);
}
int kcr_fatrelu_and_mul(const kcr_tensor* out, const kcr_tensor* input, double threshold,
                        void* stream) {
    return run_gated<ACT_FATRELU, true>(out, input, threshold, stream);
}
int kcr_gelu(const kcr_tensor* out, const kcr_tensor* input, void* stream) {
    return run_elementwise<ACT_GELU>(out, input, stream);
}
int kcr_gelu_tanh(const kcr_tensor* out, const kcr_tensor* input, void* stream) {
    return run_elementwise<ACT_GELU_TANH>(out, input, stream);
}
int kcr_gelu_new(const kcr_tensor* out, const kcr_tensor* input, void* stream) {
    return run_elementwise<ACT_GELU_NEW>(out, input, stream);
}
int kcr_gelu_fast(const kcr_tensor* out, const kcr_tensor* input, void* stream) {
    return run_elementwise<ACT_GELU_FAST>(out, input, stream);
}
int kcr_gelu_quick(const kcr_tensor* out, const kcr_tensor* input, void* stream) {
    return run_elementwise<ACT_GELU_QUICK>(out, input, stream);
}
int kcr_silu(const kcr_tensor* out, const kcr_tensor* input, void* stream) {
    return run_elementwise<ACT_SILU>(out, input, stream);
}

}  // extern "C"
