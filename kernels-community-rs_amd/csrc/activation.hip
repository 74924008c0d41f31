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
#include "common.h"

#include <algorithm>

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

template <typename T>
__device__ __forceinline__ float rnd(float v) {
    return Elem<T>::round(v);
}

// exp(x) for x in [-150, 80]: exp2 of the product x * log2(e) split into a
// rounded head and its exact residual (the head via one multiply, the residual
// via two FMAs against the two-float log2(e)), then one first-order correction
// e * (1 + residual * ln 2). Relative error about 1 ulp of f32 (v_exp_f32's own).
__device__ __forceinline__ float exp_split(float x) {
    constexpr float kLog2eHi = 1.44269502162933349609375f;  // float(log2 e)
    constexpr float kLog2eLo = 1.9259629911266175e-8f;      // log2 e - kLog2eHi
    constexpr float kLn2f = 0.693147180559945309f;
    const float h = x * kLog2eHi;
    const float lo = __builtin_fmaf(x, kLog2eLo, __builtin_fmaf(x, kLog2eHi, -h));
    const float e2 = __builtin_amdgcn_exp2f(h);
    return __builtin_fmaf(e2 * lo, kLn2f, e2);
}

// f / (1 + exp(-z)) for z > -80 (so 1 + exp(-z) < 2^116 and its reciprocal is
// a normal float) and finite f below 2^64: hardware reciprocal plus one Newton-Raphson correction of the
// quotient, within about 1 ulp of the IEEE quotient. Used for 16-bit element
// types, whose results are rounded to 8 or 11 significant bits afterwards.
__device__ __forceinline__ float div_one_plus_exp_neg(float f, float z) {
    const float d = 1.0f + exp_split(fmaxf(-z, -150.0f));
    const float r = __builtin_amdgcn_rcpf(d);
    const float q0 = f * r;
    return __builtin_fmaf(__builtin_fmaf(-d, q0, f), r, q0);
}

// tanh(u) = sign(u) (1 - s), s = 2e / (1 + e), e = exp(-2|u|) in (0, 1], with
// e = exp2(-2|u| log2 e) and the hardware reciprocal. The errors of e and s
// (a few f32 ulp, relative) reach 1 - s only as s times that, below half an ulp
// of 1 wherever s is small (|u| large, where 1 + tanh(u) cancels), so the
// reference's rounding of tanh and of 1 + tanh is reproduced there. Infinite u
// gives +-1; NaN u gives +-1 and the callers' products with the NaN input stay
// NaN.
__device__ __forceinline__ float tanh_lite(float u) {
    constexpr float kNeg2Log2e = -2.0f * 1.44269502162933349609375f;
    const float e = __builtin_amdgcn_exp2f(fmaxf(fabsf(u) * kNeg2Log2e, -300.0f));
    const float s = e * __builtin_amdgcn_rcpf(__builtin_fmaf(0.5f, e, 0.5f));  // 2e / (1 + e)
    return copysignf(1.0f - s, u);
}

// Whether the split-exp forms may stand in for the libm expression: 16-bit
// element types only (their results keep 8 or 11 significant bits).
template <typename T, int A>
constexpr bool has_fast_form() {
    // gelu_tanh: bf16 only; f16's 11-bit results near the cancellation of
    // 1 + tanh(u) resolve the few-ulp error of the exp2 / reciprocal form.
    return (sizeof(typename Elem<T>::storage) == 2 && A == ACT_SILU) ||
           (std::is_same<T, bf16_t>::value && A == ACT_GELU_TANH);
}

// Inputs the fast SiLU form covers: the split exp needs -f < 80 (no overflow of
// 1 + exp(-f), normal reciprocal), the Newton step a finite f below 2^64. The
// tails (and NaN) keep the reference expression.
template <int A>
__device__ __forceinline__ bool fast_form_covers(float f) {
    if constexpr (A == ACT_SILU) return f > -80.0f && f < 0x1p64f;
    return true;
}

template <typename T, int A, bool FAST = false>
__device__ __forceinline__ float apply_act(float f, float threshold) {
    constexpr bool kFast = FAST && has_fast_form<T, A>();
    if constexpr (A == ACT_SILU) {
        // activation.rs:42-46: f / (1 + exp(-f)); the fast form is the split exp
        // and a refined reciprocal (callers check fast_form_covers first).
        if constexpr (kFast) return rnd<T>(div_one_plus_exp_neg(f, f));
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
        // bf16: tanh from one exp2 and one reciprocal (tanh_lite), then
        // the reference's own 1 + tanh(u) and products.
        if constexpr (kFast) return rnd<T>(0.5f * f * (1.0f + tanh_lite(inner)));
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

template <typename T, int A, bool ACT_FIRST, bool FAST = false>
__device__ __forceinline__ float gated(float x, float y, float threshold) {
    if constexpr (ACT_FIRST) {
        return apply_act<T, A, FAST>(x, threshold) * y;
    } else {
        return x * apply_act<T, A, FAST>(y, threshold);
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
            // One branch per vector: the fast form when it covers every element
            // of this lane's vector (always, for ordinary data).
            bool fast = has_fast_form<T, A>();
#pragma unroll
            for (int e = 0; e < VEC; ++e) fast = fast && fast_form_covers<A>(ACT_FIRST ? x[e] : y[e]);
            if (fast) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) r[e] = gated<T, A, ACT_FIRST, true>(x[e], y[e], threshold);
            } else {
#pragma unroll
                for (int e = 0; e < VEC; ++e) r[e] = gated<T, A, ACT_FIRST>(x[e], y[e], threshold);
            }
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
        Elem<T>::store(out + i, gated<T, A, ACT_FIRST>(x, y, threshold));
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
            // The fast activation forms of the gated kernel, under the same
            // per-vector coverage check.
            bool fast = has_fast_form<T, A>();
#pragma unroll
            for (int e = 0; e < VEC; ++e) fast = fast && fast_form_covers<A>(x[e]);
            if (fast) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) r[e] = apply_act<T, A, true>(x[e], 0.0f);
            } else {
#pragma unroll
                for (int e = 0; e < VEC; ++e) r[e] = apply_act<T, A>(x[e], 0.0f);
            }
            __builtin_nontemporal_store(narrow<T>(r), out + j);
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
        Elem<T>::store(out + i, apply_act<T, A>(Elem<T>::load(in + i), 0.0f));
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
        const uint64_t need = (total + kThreads * kGatedUnroll - 1) / (kThreads * kGatedUnroll);
        const unsigned grid = static_cast<unsigned>(std::max<uint64_t>(1, std::min<uint64_t>(need, kGatedBlocks)));
        // 32-bit index math is enough when every flat index (plus one grid
        // stride of unrolled look-ahead) fits below 2^32.
        const uint64_t reach = total + static_cast<uint64_t>(grid) * kThreads * kUnroll;
        if (reach < (1ull << 32) && vpr < (1ull << 32)) {
            act_and_mul_vec<T, A, ACT_FIRST, false><<<grid, kThreads, 0, stream>>>(
                static_cast<u32x4*>(out->data), static_cast<const u32x4*>(input->data), total,
                static_cast<uint32_t>(vpr), threshold);
        } else {
            act_and_mul_vec<T, A, ACT_FIRST, true><<<grid, kThreads, 0, stream>>>(
                static_cast<u32x4*>(out->data), static_cast<const u32x4*>(input->data), total,
                static_cast<uint32_t>(vpr), threshold);
        }
    } else {
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
    if (total_elems % VEC == 0 && aligned16(out->data) && aligned16(input->data)) {
        const uint64_t total = total_elems / VEC;
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
