// RMSNorm forward, backward and weight-gradient reduction (rmsnorm crate).
//
// Reference: rmsnorm/src/device.rs:75-358 (kernels), rmsnorm/src/ops.rs:1-444
// (validation, dispatch, exports), rmsnorm/src/casting.rs:29-60 (casting modes).
//
// MI355X design (forward): rows up to 16 x 16 bytes per lane (8192 bf16 / 4096 f32
// columns) take a one-pass wave-per-row kernel. Each 64-lane wave loads its whole
// row into VGPRs with 16-byte loads, reduces the sum of squares with a wave64
// butterfly (no LDS, no barrier), and normalises straight from registers, so x is
// read from HBM exactly once and y written once. The weight row is loaded into
// registers once per wave and reused for every row the wave visits. Wider or
// misaligned rows take a block-per-row kernel that makes a second pass over the
// row (served from L2) like the reference.
//
// Backward: blocks own contiguous row ranges (one row of f32 partial weight
// gradients per block, as the reference's `dw_partial`), reduced by
// `reduce_weight_grad` in a fixed order.
#include "common.h"

#include <type_traits>

// The reference's f32 arithmetic is never fused (Rust does not contract a
// multiply and an add into an FMA), and results such as mean(x^2) + eps, i.e.
// sum * (1/n) + eps, depend on it: no contraction anywhere in this file.
#pragma clang fp contract(off)

namespace kcr {

enum Mode : int { MODE_LLAMA = 0, MODE_GEMMA = 1, MODE_NONE = 2 };

// Casting-mode flags of rmsnorm/src/casting.rs:44-60.
template <int M>
struct Casting {
    static constexpr bool input_dtype_math = (M == MODE_NONE);
    static constexpr bool round_x_hat = (M != MODE_GEMMA);
    static constexpr bool round_weight_grad = (M == MODE_LLAMA);
};

// f32 -> T -> f32, from the rounded f32 value.
template <typename T>
__device__ __forceinline__ float rnd(float v) {
    return Elem<T>::round(as_f32(v));
}

// Stores an f32 result as T, from the rounded f32 value.
template <typename T>
__device__ __forceinline__ void store_rn(T* p, float v) {
    Elem<T>::store(p, as_f32(v));
}

template <typename T>
constexpr int vec_of() {
    return 16 / sizeof(typename Elem<T>::storage);
}

// 16 bytes of T (8 x 16-bit or 4 x f32) widened into f[0..VEC).
template <typename T>
__device__ __forceinline__ void widen16(const u32x4& w, float* f) {
    if constexpr (sizeof(typename Elem<T>::storage) == 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) f[i] = __uint_as_float(w[i]);
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[2 * i] = Elem<T>::to_f32(w[i] & 0xffffu);
            f[2 * i + 1] = Elem<T>::to_f32(w[i] >> 16);
        }
    }
}

template <typename T>
__device__ __forceinline__ u32x4 narrow16(const float* f) {
    u32x4 w;
    if constexpr (sizeof(typename Elem<T>::storage) == 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = __float_as_uint(f[i]);
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = pack_pair<T>(as_f32(f[2 * i]), as_f32(f[2 * i + 1]));
    }
    return w;
}

// rstd = 1 / sqrt(mean(x^2) + eps), device.rs:147-153. mean(x^2) is the f32
// product sum_sq * inv_n and the eps add is f32 as in the reference; the inverse
// square root is evaluated in f64 and rounded once to f32, i.e. the correctly
// rounded f32 value (the reference calls libdevice's rsqrtf, which approximates
// that value).
__device__ __forceinline__ float rsqrt_rn(float v) {
    return static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(v)));
}

template <typename X, int M>
__device__ __forceinline__ float row_rstd(float sum_sq, float inv_n, float eps) {
    const float mean_square = sum_sq * inv_n;
    if constexpr (Casting<M>::input_dtype_math) {
        return rnd<X>(rsqrt_rn(rnd<X>(mean_square) + rnd<X>(eps)));
    } else {
        return rsqrt_rn(mean_square + eps);
    }
}

// y = x_hat * (offset + w), device.rs:161-179.
template <typename X, typename W, int M, bool AFFINE>
__device__ __forceinline__ float normalize(float x, float w, float rstd, float offset) {
    const float xr = x * rstd;
    const float x_hat = Casting<M>::round_x_hat ? rnd<X>(xr) : xr;
    if constexpr (!AFFINE) {
        return x_hat;
    } else {
        const float factor =
            Casting<M>::input_dtype_math ? rnd<W>(rnd<X>(offset) + w) : offset + w;
        return x_hat * factor;
    }
}

// ---------------------------------------------------------------------------
// The sum of squares of a row, in the reference's order.
//
// The reference (device.rs:41-63, 113-145) runs T = block_threads(n) threads
// per row (ops.rs:98-106). With 16-byte access ("vectorized", ops.rs:108-115)
// thread t owns the 8-element groups t, t + T, t + 2T, ... of the first
// floor(n / 8) * 8 columns and then the single columns tail + t, tail + t + T,
// ...; without it, the single columns t, t + T, .... Its partial is
//   S(g0) + S(g1) + ... + x_c * x_c + ...,   S(g) = (((q0 + q1) + q2) ... + q7),
// every product and sum rounded to f32 (no fused multiply-add). The partials
// of each 32-thread warp are reduced by a butterfly with lane distances 16, 8,
// 4, 2, 1, and the T / 32 warp sums by the same butterfly over 32 slots of
// which the first T / 32 hold the sums (the rest zero). The kernels below
// reproduce that order exactly, so the row's sum, rstd and y are the same bits
// whichever kernel runs.
// ---------------------------------------------------------------------------

// One f32 product added to a running sum, rounded twice.
__device__ __forceinline__ float add_square(float sum, float v) { return sum + v * v; }

// S(g) of 8 widened values.
__device__ __forceinline__ float group_squares(const float* f) {
    float s = f[0] * f[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) s = s + f[i] * f[i];
    return s;
}

// v + (value of the lane at distance D within the lane's 32-lane half).
template <int D>
__device__ __forceinline__ float add_xor32(float v) {
    // ds_swizzle bit-mask mode: and_mask 0x1f, xor_mask D (within 32 lanes).
    const int other = __builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1f | (D << 10));
    return v + __int_as_float(other);
}

// The 32-lane butterfly of one warp: every lane of a 32-lane half ends with
// the half's sum in the reference's pairing.
__device__ __forceinline__ float warp32_sum(float v) {
    v = add_xor32<16>(v);
    v = add_xor32<8>(v);
    v = add_xor32<4>(v);
    v = add_xor32<2>(v);
    return add_xor32<1>(v);
}

// The block-level butterfly over NW warp sums (NW in {4, 8, 16, 32}): slots
// NW..31 are zero and adding them changes nothing (the sums are >= +0), so the
// steps with distance >= NW are skipped.
template <int NW>
__device__ __forceinline__ float warp_tree(float (&p)[NW]) {
#pragma unroll
    for (int d = NW / 2; d >= 1; d /= 2) {
#pragma unroll
        for (int i = 0; i < d; ++i) p[i] = p[i] + p[i + d];
    }
    return p[0];
}

// Widens the 8-element group at `p` (16-byte aligned) to f32.
template <typename X>
__device__ __forceinline__ void load_group(const X* p, float (&f)[8]) {
    const u32x4* v = reinterpret_cast<const u32x4*>(p);
    if constexpr (sizeof(typename Elem<X>::storage) == 4) {
        widen16<float>(v[0], f);
        widen16<float>(v[1], f + 4);
    } else {
        widen16<X>(v[0], f);
    }
}

template <typename X>
__device__ __forceinline__ void store_group(X* p, const float (&f)[8]) {
    u32x4* v = reinterpret_cast<u32x4*>(p);
    if constexpr (sizeof(typename Elem<X>::storage) == 4) {
        v[0] = narrow16<float>(f);
        v[1] = narrow16<float>(f + 4);
    } else {
        v[0] = narrow16<X>(f);
    }
}

constexpr int kWaves = 4;  // waves per block of the wave-per-row kernel

// One wave per row, the row held in registers. Lane l holds the 8-element
// groups l + 64 c (c < CHUNKS), each as 16 bytes (16-bit X) or 32 bytes (f32).
// The reference thread owning group g is g mod T, so with SLOTS = T / 64 the
// lane's group c belongs to thread l + 64 (c mod SLOTS), warp 2 (c mod SLOTS) +
// (l >= 32): the lane keeps one partial per slot and the 32-lane butterflies
// give the warp sums. Requires n % 8 == 0, 16-byte aligned tensors and (with
// AFFINE) a weight of X's type or f32.
template <typename X, typename W, int M, bool AFFINE, int CHUNKS, int SLOTS, bool WLDS>
__global__ void __launch_bounds__(64 * kWaves) rms_fwd_wave(
    X* __restrict__ y, float* __restrict__ rstd_out, const X* __restrict__ x,
    const W* __restrict__ weight, uint32_t rows, uint32_t groups, float inv_n, float eps,
    float offset) {
    constexpr int XV = sizeof(typename Elem<X>::storage) == 4 ? 2 : 1;  // 16-byte vectors per group
    constexpr int WV = sizeof(typename Elem<W>::storage) == 4 ? 2 : 1;
    constexpr int NW = 2 * SLOTS;
    const int lane = threadIdx.x & 63;
    const uint32_t wave = blockIdx.x * kWaves + (threadIdx.x >> 6);
    const uint32_t waves = gridDim.x * kWaves;
    const uint32_t n = groups * 8;

    u32x4 wv[AFFINE && !WLDS ? CHUNKS * WV : 1];
    __shared__ u32x4 w_lds[AFFINE && WLDS ? CHUNKS * WV * 64 : 1];
    if constexpr (AFFINE) {
        const u32x4* wp = reinterpret_cast<const u32x4*>(weight);
        if constexpr (WLDS) {
            // The weight staged once per block, lane-contiguous per chunk.
            for (uint32_t i = threadIdx.x; i < CHUNKS * WV * 64u; i += 64u * kWaves) {
                const uint32_t c = i / (64u * WV), rest = i - c * 64u * WV;
                const uint32_t h = rest / 64u, l = rest - h * 64u;
                const uint32_t g = l + 64u * c;
                if (g < groups) w_lds[i] = wp[g * WV + h];
            }
            __syncthreads();
        } else {
#pragma unroll
            for (int c = 0; c < CHUNKS; ++c) {
                const uint32_t g = lane + 64u * c;
#pragma unroll
                for (int h = 0; h < WV; ++h) {
                    if (g < groups) wv[c * WV + h] = wp[g * WV + h];
                }
            }
        }
    }
    auto weight_vec = [&](int c, int h) -> u32x4 {
        if constexpr (WLDS) {
            return w_lds[(c * WV + h) * 64 + lane];
        } else {
            return wv[c * WV + h];
        }
    };

    // Rows are dealt to waves round-robin; the next row's loads are issued
    // before the current row is reduced and written, so every wave keeps a
    // whole row of reads in flight.
    auto load_row = [&](uint32_t r, u32x4 (&dst)[CHUNKS * XV]) {
        const u32x4* xr = reinterpret_cast<const u32x4*>(x + static_cast<uint64_t>(r) * n);
#pragma unroll
        for (int c = 0; c < CHUNKS; ++c) {
            const uint32_t g = lane + 64u * c;
#pragma unroll
            for (int h = 0; h < XV; ++h) {
                if (g < groups) dst[c * XV + h] = __builtin_nontemporal_load(xr + g * XV + h);
            }
        }
    };
    auto widen_x = [&](const u32x4 (&src)[CHUNKS * XV], int c, float (&f)[8]) {
        if constexpr (XV == 2) {
            widen16<float>(src[2 * c], f);
            widen16<float>(src[2 * c + 1], f + 4);
        } else {
            widen16<X>(src[c], f);
        }
    };
    u32x4 xv[CHUNKS * XV];
    if (wave < rows) load_row(wave, xv);
    for (uint32_t row = wave; row < rows; row += waves) {
        u32x4 xn[CHUNKS * XV];
        if (row + waves < rows) load_row(row + waves, xn);
        float part[SLOTS];
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) part[s] = 0.0f;
#pragma unroll
        for (int c = 0; c < CHUNKS; ++c) {
            if (lane + 64u * c < groups) {
                float f[8];
                widen_x(xv, c, f);
                part[c % SLOTS] = part[c % SLOTS] + group_squares(f);
            }
        }
        // Warp sums: slot s of the lower half is warp 2s, of the upper half 2s + 1.
        float ws[NW];
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) {
            const float own = s < CHUNKS ? warp32_sum(part[s]) : 0.0f;
            const float other = __shfl_xor(own, 32);
            const bool upper = lane >= 32;
            ws[2 * s] = upper ? other : own;
            ws[2 * s + 1] = upper ? own : other;
        }
        const float rstd = row_rstd<X, M>(warp_tree<NW>(ws), inv_n, eps);
        if (lane == 0) rstd_out[row] = rstd;
        X* yr = y + static_cast<uint64_t>(row) * n;
#pragma unroll
        for (int c = 0; c < CHUNKS; ++c) {
            const uint32_t g = lane + 64u * c;
            if (g < groups) {
                float f[8], w[8], o[8];
                widen_x(xv, c, f);
                if constexpr (AFFINE) {
                    if constexpr (WV == 2) {
                        widen16<float>(weight_vec(c, 0), w);
                        widen16<float>(weight_vec(c, 1), w + 4);
                    } else {
                        widen16<W>(weight_vec(c, 0), w);
                    }
                }
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    o[e] = normalize<X, W, M, AFFINE>(f[e], AFFINE ? w[e] : 0.0f, rstd, offset);
                u32x4* yv = reinterpret_cast<u32x4*>(yr) + g * XV;
                if constexpr (XV == 2) {
                    __builtin_nontemporal_store(narrow16<float>(o), yv);
                    __builtin_nontemporal_store(narrow16<float>(o + 4), yv + 1);
                } else {
                    __builtin_nontemporal_store(narrow16<X>(o), yv);
                }
            }
        }
#pragma unroll
        for (int c = 0; c < CHUNKS * XV; ++c) xv[c] = xn[c];
    }
}

// Block per row with the reference's T = blockDim.x threads and its column
// assignment (groups when `vectorized`, then single columns); two passes over
// the row (the second mostly from L2). NW = T / 32 warp sums.
template <typename X, typename W, int M, bool AFFINE, int NW>
__global__ void __launch_bounds__(32 * NW) rms_fwd_block(X* __restrict__ y, float* __restrict__ rstd_out,
                                                         const X* __restrict__ x,
                                                         const W* __restrict__ weight, uint32_t n,
                                                         uint32_t vectorized, float inv_n, float eps,
                                                         float offset) {
    __shared__ float warp_sums[NW];
    constexpr uint32_t T = 32 * NW;
    const uint64_t row = blockIdx.x;
    const X* xr = x + row * n;
    X* yr = y + row * n;
    const uint32_t t = threadIdx.x;
    const uint32_t tail = vectorized ? n / 8 * 8 : 0;
    float sum = 0.0f;
    for (uint32_t col = 8 * t; col < tail; col += 8 * T) {
        float f[8];
        load_group<X>(xr + col, f);
        sum = sum + group_squares(f);
    }
    for (uint32_t col = tail + t; col < n; col += T) sum = add_square(sum, Elem<X>::load(xr + col));
    sum = warp32_sum(sum);
    if ((t & 31) == 0) warp_sums[t >> 5] = sum;
    __syncthreads();
    float p[NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) p[i] = warp_sums[i];
    const float rstd = row_rstd<X, M>(warp_tree<NW>(p), inv_n, eps);
    if (t == 0) rstd_out[row] = rstd;
    for (uint32_t col = 8 * t; col < tail; col += 8 * T) {
        float f[8], w[8], o[8];
        load_group<X>(xr + col, f);
        if constexpr (AFFINE) load_group<W>(weight + col, w);
#pragma unroll
        for (int e = 0; e < 8; ++e)
            o[e] = normalize<X, W, M, AFFINE>(f[e], AFFINE ? w[e] : 0.0f, rstd, offset);
        store_group<X>(yr + col, o);
    }
    for (uint32_t col = tail + t; col < n; col += T) {
        const float w = AFFINE ? Elem<W>::load(weight + col) : 0.0f;
        store_rn<X>(yr + col, normalize<X, W, M, AFFINE>(Elem<X>::load(xr + col), w, rstd, offset));
    }
}

// Gradients of the forward pass, device.rs:228-335:
//   m  = dy * (offset + w);  dx = rstd * m + rstd * (-(rstd^2 / n) * dot(m, x) * x)
//   dw_partial[block, :] = sum over the block's rows of dy * x_hat
template <typename X, typename W, int M, bool AFFINE>
__global__ void __launch_bounds__(1024) rms_bwd_block(X* dx, float* __restrict__ dw_partial,
                                                      const X* dy, const X* __restrict__ x,
                                                      const W* __restrict__ weight,
                                                      const float* __restrict__ rstd,
                                                      uint32_t rows, uint32_t n, float inv_n,
                                                      float offset) {
    __shared__ float partial[16];
    const uint32_t per_block = (rows + gridDim.x - 1) / gridDim.x;
    uint32_t row = blockIdx.x * per_block;
    const uint32_t row_end = min(row + per_block, rows);
    float* dw_row = dw_partial + static_cast<uint64_t>(blockIdx.x) * n;
    if constexpr (AFFINE) {
        for (uint32_t c = threadIdx.x; c < n; c += blockDim.x) dw_row[c] = 0.0f;
    }
    const int nw = blockDim.x >> 6;
    for (; row < row_end; ++row) {
        const uint64_t base = static_cast<uint64_t>(row) * n;
        const float r = rstd[row];
        float dot = 0.0f;
        for (uint32_t c = threadIdx.x; c < n; c += blockDim.x) {
            float g = Elem<X>::load(dy + base + c);
            if constexpr (AFFINE) g *= Elem<W>::load(weight + c) + offset;
            dot += g * Elem<X>::load(x + base + c);
        }
        dot = wave_sum(dot);
        if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = dot;
        __syncthreads();
        float total = (threadIdx.x & 63) < nw ? partial[threadIdx.x & 63] : 0.0f;
        total = wave_sum(total);
        const float correction = -inv_n * r * r * total;
        for (uint32_t c = threadIdx.x; c < n; c += blockDim.x) {
            const float g0 = Elem<X>::load(dy + base + c);
            const float xv = Elem<X>::load(x + base + c);
            float g = g0;
            if constexpr (AFFINE) g *= Elem<W>::load(weight + c) + offset;
            store_rn<X>(dx + base + c, r * g + r * (correction * xv));
            if constexpr (AFFINE) {
                const bool rw = Casting<M>::round_weight_grad;
                const float x_hat = rw ? rnd<X>(xv * r) : xv * r;
                const float contrib = rw ? rnd<X>(g0 * x_hat) : g0 * x_hat;
                dw_row[c] += contrib;
            }
        }
        // The next row reuses `partial`.
        __syncthreads();
    }
}

// Backward with one wave per partial-gradient row: the wave owns rows
// [part * per, (part + 1) * per), reads each row's dy and x once with 16-byte
// loads (CHUNKS vectors per lane), and keeps the row's fp32 dw contributions in
// registers, summed over its rows in order. Same arithmetic and rounding points
// as rms_bwd_block. Requires 16-bit x, a weight of x's type or f32, n % 8 == 0
// and 16-byte aligned tensors. dy may alias dx (each row is read whole before
// it is written).
template <typename X, typename W, int M, bool AFFINE, int CHUNKS>
__global__ void __launch_bounds__(64 * kWaves) rms_bwd_wave(u32x4* dx, float* __restrict__ dw_partial,
                                                           const u32x4* dy, const u32x4* __restrict__ x,
                                                           const u32x4* __restrict__ weight,
                                                           const float* __restrict__ rstd, uint32_t rows,
                                                           uint32_t nvec, uint32_t parts, float inv_n,
                                                           float offset) {
    constexpr int VEC = vec_of<X>();
    static_assert(VEC == 8, "16-bit element types");
    // f32 weight: two 16-byte weight vectors per x vector.
    constexpr int WPV = sizeof(typename Elem<W>::storage) == 4 ? 2 : 1;
    const int lane = threadIdx.x & 63;
    const uint32_t part = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (part >= parts) return;
    const uint32_t per = (rows + parts - 1) / parts;
    const uint64_t r0 = static_cast<uint64_t>(part) * per;
    const uint64_t r1 = r0 + per < rows ? r0 + per : rows;

    u32x4 wv[CHUNKS * WPV];
    if constexpr (AFFINE) {
#pragma unroll
        for (int c = 0; c < CHUNKS; ++c) {
            const uint32_t v = lane + 64u * c;
#pragma unroll
            for (int h = 0; h < WPV; ++h) {
                if (v < nvec) wv[c * WPV + h] = weight[v * WPV + h];
            }
        }
    }
    auto widen_w = [&](int c, float* wf) __attribute__((always_inline)) {
        if constexpr (WPV == 2) {
            widen16<float>(wv[2 * c], wf);
            widen16<float>(wv[2 * c + 1], wf + 4);
        } else {
            widen16<W>(wv[c], wf);
        }
    };
    float acc[AFFINE ? CHUNKS * VEC : 1];
#pragma unroll
    for (int i = 0; i < (AFFINE ? CHUNKS * VEC : 1); ++i) acc[i] = 0.0f;

    // The next row's dy and x are loaded before the current row is reduced and
    // written (a different row, so this holds with dy aliasing dx too).
    auto load_row = [&](uint64_t row, u32x4 (&g)[CHUNKS], u32x4 (&xr)[CHUNKS]) __attribute__((always_inline)) {
        const uint64_t base = row * nvec;
#pragma unroll
        for (int c = 0; c < CHUNKS; ++c) {
            const uint32_t v = lane + 64u * c;
            if (v < nvec) {
                g[c] = dy[base + v];
                xr[c] = __builtin_nontemporal_load(x + base + v);
            }
        }
    };
    u32x4 gv[CHUNKS], xv[CHUNKS];
    if (r0 < r1) load_row(r0, gv, xv);
    for (uint64_t row = r0; row < r1; ++row) {
        const uint64_t base = row * nvec;
        u32x4 gn[CHUNKS], xn[CHUNKS];
        if (row + 1 < r1) load_row(row + 1, gn, xn);
        const float r = rstd[row];
        float dot = 0.0f;
#pragma unroll
        for (int c = 0; c < CHUNKS; ++c) {
            const uint32_t v = lane + 64u * c;
            if (v < nvec) {
                float g[VEC], xf[VEC], wf[VEC];
                widen16<X>(gv[c], g);
                widen16<X>(xv[c], xf);
                if constexpr (AFFINE) widen_w(c, wf);
#pragma unroll
                for (int e = 0; e < VEC; ++e) dot += (AFFINE ? g[e] * (wf[e] + offset) : g[e]) * xf[e];
            }
        }
        dot = wave_sum(dot);
        const float correction = -inv_n * r * r * dot;
#pragma unroll
        for (int c = 0; c < CHUNKS; ++c) {
            const uint32_t v = lane + 64u * c;
            if (v < nvec) {
                float g[VEC], xf[VEC], wf[VEC], o[VEC];
                widen16<X>(gv[c], g);
                widen16<X>(xv[c], xf);
                if constexpr (AFFINE) widen_w(c, wf);
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    const float gg = AFFINE ? g[e] * (wf[e] + offset) : g[e];
                    o[e] = r * gg + r * (correction * xf[e]);
                    if constexpr (AFFINE) {
                        const bool rw = Casting<M>::round_weight_grad;
                        const float x_hat = rw ? rnd<X>(xf[e] * r) : xf[e] * r;
                        acc[c * VEC + e] += rw ? rnd<X>(g[e] * x_hat) : g[e] * x_hat;
                    }
                }
                __builtin_nontemporal_store(narrow16<X>(o), dx + base + v);
            }
        }
#pragma unroll
        for (int c = 0; c < CHUNKS; ++c) {
            gv[c] = gn[c];
            xv[c] = xn[c];
        }
    }
    if constexpr (AFFINE) {
        float4* dwr = reinterpret_cast<float4*>(dw_partial + static_cast<uint64_t>(part) * nvec * VEC);
#pragma unroll
        for (int c = 0; c < CHUNKS; ++c) {
            const uint32_t v = lane + 64u * c;
            if (v < nvec) {
                const float* a = acc + c * VEC;
                dwr[2 * v] = float4{a[0], a[1], a[2], a[3]};
                dwr[2 * v + 1] = float4{a[4], a[5], a[6], a[7]};
            }
        }
    }
}

// The same backward with the columns of each partial row split over two waves
// (one 128-thread block per partial row): each wave holds half the row, the
// row's dot product is the sum of the two halves' wave sums exchanged through
// LDS (one barrier per row, the slot alternating with the row's parity), and
// each wave keeps and writes its half of the dw partial. Half the registers of
// rms_bwd_wave (for 8 chunks: 426 -> ~150), so more waves fit per SIMD.
template <typename X, typename W, int M, bool AFFINE, int CHUNKS>
__global__ void __launch_bounds__(128) rms_bwd_split(u32x4* dx, float* __restrict__ dw_partial,
                                                     const u32x4* dy, const u32x4* __restrict__ x,
                                                     const u32x4* __restrict__ weight,
                                                     const float* __restrict__ rstd, uint32_t rows,
                                                     uint32_t nvec, uint32_t parts, float inv_n,
                                                     float offset) {
    constexpr int VEC = vec_of<X>();
    static_assert(VEC == 8, "16-bit element types");
    static_assert(CHUNKS % 2 == 0, "two halves");
    constexpr int HC = CHUNKS / 2;
    constexpr int WPV = sizeof(typename Elem<W>::storage) == 4 ? 2 : 1;
    __shared__ float dots[2][2];
    const int lane = threadIdx.x & 63;
    const int half = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t part = blockIdx.x;
    if (part >= parts) return;  // block-uniform
    const uint32_t per = (rows + parts - 1) / parts;
    const uint64_t r0 = static_cast<uint64_t>(part) * per;
    const uint64_t r1 = r0 + per < rows ? r0 + per : rows;
    // Vector index of this lane's chunk c.
    auto vec_at = [&](int c) { return static_cast<uint32_t>(lane + 64 * (half * HC + c)); };

    u32x4 wv[AFFINE ? HC * WPV : 1];
    if constexpr (AFFINE) {
#pragma unroll
        for (int c = 0; c < HC; ++c) {
            const uint32_t v = vec_at(c);
#pragma unroll
            for (int h = 0; h < WPV; ++h) {
                if (v < nvec) wv[c * WPV + h] = weight[v * WPV + h];
            }
        }
    }
    auto widen_w = [&](int c, float* wf) __attribute__((always_inline)) {
        if constexpr (WPV == 2) {
            widen16<float>(wv[2 * c], wf);
            widen16<float>(wv[2 * c + 1], wf + 4);
        } else {
            widen16<W>(wv[c], wf);
        }
    };
    float acc[AFFINE ? HC * VEC : 1];
#pragma unroll
    for (int i = 0; i < (AFFINE ? HC * VEC : 1); ++i) acc[i] = 0.0f;

    auto load_row = [&](uint64_t row, u32x4 (&g)[HC], u32x4 (&xr)[HC]) __attribute__((always_inline)) {
        const uint64_t base = row * nvec;
#pragma unroll
        for (int c = 0; c < HC; ++c) {
            const uint32_t v = vec_at(c);
            if (v < nvec) {
                g[c] = dy[base + v];
                xr[c] = __builtin_nontemporal_load(x + base + v);
            }
        }
    };
    u32x4 gv[HC], xv[HC];
    if (r0 < r1) load_row(r0, gv, xv);
    for (uint64_t row = r0; row < r1; ++row) {
        const uint64_t base = row * nvec;
        u32x4 gn[HC], xn[HC];
        if (row + 1 < r1) load_row(row + 1, gn, xn);
        const float r = rstd[row];
        float dot = 0.0f;
#pragma unroll
        for (int c = 0; c < HC; ++c) {
            if (vec_at(c) < nvec) {
                float g[VEC], xf[VEC], wf[VEC];
                widen16<X>(gv[c], g);
                widen16<X>(xv[c], xf);
                if constexpr (AFFINE) widen_w(c, wf);
#pragma unroll
                for (int e = 0; e < VEC; ++e) dot += (AFFINE ? g[e] * (wf[e] + offset) : g[e]) * xf[e];
            }
        }
        dot = wave_sum(dot);
        const int slot = static_cast<int>(row & 1);
        if (lane == 0) dots[slot][half] = dot;
        __syncthreads();
        const float total = dots[slot][0] + dots[slot][1];
        const float correction = -inv_n * r * r * total;
#pragma unroll
        for (int c = 0; c < HC; ++c) {
            const uint32_t v = vec_at(c);
            if (v < nvec) {
                float g[VEC], xf[VEC], wf[VEC], o[VEC];
                widen16<X>(gv[c], g);
                widen16<X>(xv[c], xf);
                if constexpr (AFFINE) widen_w(c, wf);
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    const float gg = AFFINE ? g[e] * (wf[e] + offset) : g[e];
                    o[e] = r * gg + r * (correction * xf[e]);
                    if constexpr (AFFINE) {
                        const bool rw = Casting<M>::round_weight_grad;
                        const float x_hat = rw ? rnd<X>(xf[e] * r) : xf[e] * r;
                        acc[c * VEC + e] += rw ? rnd<X>(g[e] * x_hat) : g[e] * x_hat;
                    }
                }
                __builtin_nontemporal_store(narrow16<X>(o), dx + base + v);
            }
        }
#pragma unroll
        for (int c = 0; c < HC; ++c) {
            gv[c] = gn[c];
            xv[c] = xn[c];
        }
    }
    if constexpr (AFFINE) {
        float4* dwr = reinterpret_cast<float4*>(dw_partial + static_cast<uint64_t>(part) * nvec * VEC);
#pragma unroll
        for (int c = 0; c < HC; ++c) {
            const uint32_t v = vec_at(c);
            if (v < nvec) {
                const float* a = acc + c * VEC;
                dwr[2 * v] = float4{a[0], a[1], a[2], a[3]};
                dwr[2 * v + 1] = float4{a[4], a[5], a[6], a[7]};
            }
        }
    }
}

// dw[c] = sum_b dw_partial[b, c] in a fixed order, rounded to W (device.rs:339-358).
// One block per 32 columns: each half-wave covers the 32 columns (128-byte
// rows), the two halves taking alternate partial rows. Each of the 16 waves
// sums a contiguous run of partial rows (8 loads in flight per lane), the
// halves' sums are added, and wave 0 adds the 16 run sums in order. The order
// is fixed, so results repeat bit for bit (it differs from one sequential
// chain only by fp32 rounding).
constexpr int kReduceWaves = 16;
constexpr int kReduceCols = 32;  // columns per block: a half-wave each, 128-byte rows
template <typename W>
__global__ void __launch_bounds__(64 * kReduceWaves) reduce_weight_grad(W* __restrict__ dw,
                                                                        const float* __restrict__ dw_partial,
                                                                        uint32_t blocks, uint32_t n) {
    __shared__ float run_sum[kReduceWaves][kReduceCols];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int col = lane & (kReduceCols - 1);
    const int sub = lane / kReduceCols;  // the two half-waves take alternate partial rows
    const uint32_t c = blockIdx.x * kReduceCols + col;
    // 64-bit so that blocks near 2^32 cannot wrap the run length to zero.
    const uint64_t per = (static_cast<uint64_t>(blocks) + kReduceWaves - 1) / kReduceWaves;
    const uint32_t b0 = static_cast<uint32_t>(min(static_cast<uint64_t>(wave) * per, static_cast<uint64_t>(blocks)));
    const uint32_t b1 = static_cast<uint32_t>(min(static_cast<uint64_t>(b0) + per, static_cast<uint64_t>(blocks)));
    float sum = 0.0f;
    if (c < n) {
        uint32_t b = b0 + sub;
        for (; b + 14 < b1; b += 16) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = dw_partial[static_cast<uint64_t>(b + 2 * u) * n + c];
#pragma unroll
            for (int u = 0; u < 8; ++u) sum += v[u];
        }
        for (; b < b1; b += 2) sum += dw_partial[static_cast<uint64_t>(b) * n + c];
    }
    sum += __shfl_xor(sum, kReduceCols, 64);
    if (sub == 0) run_sum[wave][col] = sum;
    __syncthreads();
    if (wave == 0 && sub == 0 && c < n) {
        float total = 0.0f;
#pragma unroll
        for (int w = 0; w < kReduceWaves; ++w) total += run_sum[w][col];
        store_rn<W>(dw + c, total);
    }
}

namespace {

constexpr int64_t kMaxCols = 65536;
constexpr int64_t kMaxGridX = 2147483647;

int parse_mode(const char* name) {
    const std::string s = name ? name : "";
    if (s == "llama") return MODE_LLAMA;
    if (s == "gemma") return MODE_GEMMA;
    if (s == "none") return MODE_NONE;
    throw value_error("invalid casting mode \"" + s +
                      "\", expected \"llama\", \"gemma\" or \"none\"");
}

// rows_and_cols of rmsnorm/src/ops.rs:57-74.
void rows_and_cols(const kcr_tensor* x, int64_t& rows, int64_t& n) {
    if (x->ndim == 0) throw value_error("x must have at least one dimension");
    n = x->shape[x->ndim - 1];
    if (n > kMaxCols) {
        throw value_error("the hidden size of x is " + std::to_string(n) + ", at most " +
                          std::to_string(kMaxCols) + " is supported");
    }
    rows = 1;
    for (int i = 0; i + 1 < x->ndim; ++i) rows *= x->shape[i];
    if (rows > kMaxGridX) {
        throw value_error("x has " + std::to_string(rows) + " rows, at most " +
                          std::to_string(kMaxGridX) + " are supported");
    }
}

void check_like(const kcr_tensor* t, const kcr_tensor* like, const char* name,
                const char* like_name) {
    if (shape_of(*t) != shape_of(*like) || t->dtype != like->dtype) {
        throw value_error(std::string(name) + " must have the shape and dtype of " + like_name);
    }
}

void check_f32(const kcr_tensor* t, int64_t count, const char* name) {
    if (t->dtype != KCR_FLOAT32 || numel(*t) != count) {
        throw value_error(std::string(name) + " must be a float32 tensor with " +
                          std::to_string(count) + " elements");
    }
}

void check_weight(const kcr_tensor* w, int64_t n) {
    if (w && (w->ndim != 1 || w->shape[0] != n)) {
        throw value_error("weight must have shape [" + std::to_string(n) + "], got " +
                          shape_string(*w));
    }
}

void check_input_dtype(const kcr_tensor* x) {
    if (x->dtype != KCR_FLOAT16 && x->dtype != KCR_BFLOAT16 && x->dtype != KCR_FLOAT32) {
        throw value_error("unsupported dtype, expected float16, bfloat16 or float32");
    }
}

void check_weight_dtype(const kcr_tensor* w, const kcr_tensor* x) {
    if (w && w->dtype != x->dtype && w->dtype != KCR_FLOAT32) {
        throw value_error("weight must have the dtype of x or be float32");
    }
}

void check_contiguous(const kcr_tensor* t, const char* name) {
    if (t && !is_contiguous(*t)) throw value_error(std::string(name) + " must be contiguous");
    require_device(t, name);
}

// Threads per block of the reference for rows of n elements (ops.rs:98-106);
// the forward kernels reproduce its reduction order for this count.
unsigned block_threads(int64_t n) {
    if (n < 2048) return 128;
    if (n < 8192) return 256;
    if (n < 32768) return 512;
    return 1024;
}

struct Fwd {
    const kcr_tensor *y, *rstd, *x, *w;
    int64_t rows, n;
    float eps, offset;
    hipStream_t stream;
};

template <typename X, typename W, int M, bool AFFINE, int CHUNKS, int SLOTS>
void launch_wave(const Fwd& f, uint32_t groups) {
    const uint64_t waves_needed = static_cast<uint64_t>(f.rows);
    uint64_t blocks = (waves_needed + kWaves - 1) / kWaves;
    // Each wave loops over rows with the next row prefetched; shorter rows run
    // six blocks (24 waves) per CU (one wave per row measured 50 us against
    // 45.5 us for this at 16384 x 4096 bf16 with the weight in registers).
    // Rows of 8 or more chunks (n >= 4096 at 16 bits) stage the weight in LDS
    // instead of registers (184 -> 122 VGPRs at n = 4096 bf16, 2 -> 4 waves per
    // SIMD) and run up to 16 blocks per CU: 44.0 us against 44.9 us for the
    // register weight at 6 blocks per CU (16384 x 4096 bf16; 12 / 24 / one-shot
    // grids 44.6 / 44.1 / 44.1 us).
    constexpr bool WLDS = CHUNKS >= 8;
    const uint64_t cap = (WLDS ? 16ull : 6ull) * compute_units();
    if (blocks > cap) blocks = cap;
    rms_fwd_wave<X, W, M, AFFINE, CHUNKS, SLOTS, WLDS><<<static_cast<unsigned>(blocks), 64 * kWaves, 0, f.stream>>>(
        static_cast<X*>(f.y->data), static_cast<float*>(f.rstd->data),
        static_cast<const X*>(f.x->data),
        static_cast<const W*>(AFFINE ? f.w->data : f.x->data), static_cast<uint32_t>(f.rows),
        groups, 1.0f / static_cast<float>(f.n), f.eps, f.offset);
}

template <typename X, typename W, int M, bool AFFINE, int CHUNKS>
void launch_wave_slots(const Fwd& f, uint32_t groups) {
    switch (block_threads(f.n)) {
        case 128: return launch_wave<X, W, M, AFFINE, CHUNKS, 2>(f, groups);
        case 256: return launch_wave<X, W, M, AFFINE, CHUNKS, 4>(f, groups);
        default: return launch_wave<X, W, M, AFFINE, CHUNKS, 8>(f, groups);
    }
}

template <typename X, typename W, int M, bool AFFINE>
void launch_fwd(const Fwd& f) {
    // The reference's 16-byte condition (ops.rs:108-115): rows of a multiple
    // of 16 bytes and 16-byte aligned x, y and weight.
    const bool vectorized = (f.n * sizeof(typename Elem<X>::storage)) % 16 == 0 &&
                            aligned16(f.x->data) && aligned16(f.y->data) &&
                            (!AFFINE || aligned16(f.w->data));
    // Registers hold at most 16 x 16 bytes of the row per lane (8192 16-bit or
    // 4096 f32 columns); the slot count T / 64 is at most 8 there.
    constexpr int kMaxChunks = sizeof(typename Elem<X>::storage) == 4 ? 8 : 16;
    if (vectorized && f.n % 8 == 0 && f.n <= 64 * 8 * kMaxChunks) {
        const uint32_t groups = static_cast<uint32_t>(f.n / 8);
        const uint32_t chunks = (groups + 63) / 64;
        if (chunks <= 1) return launch_wave_slots<X, W, M, AFFINE, 1>(f, groups);
        if (chunks <= 2) return launch_wave_slots<X, W, M, AFFINE, 2>(f, groups);
        if (chunks <= 4) return launch_wave_slots<X, W, M, AFFINE, 4>(f, groups);
        if (chunks <= 8) return launch_wave_slots<X, W, M, AFFINE, 8>(f, groups);
        if constexpr (kMaxChunks == 16) return launch_wave_slots<X, W, M, AFFINE, 16>(f, groups);
    }
    auto go = [&](auto nw_tag) {
        constexpr int NW = decltype(nw_tag)::value;
        rms_fwd_block<X, W, M, AFFINE, NW><<<static_cast<unsigned>(f.rows), 32 * NW, 0, f.stream>>>(
            static_cast<X*>(f.y->data), static_cast<float*>(f.rstd->data),
            static_cast<const X*>(f.x->data), static_cast<const W*>(AFFINE ? f.w->data : f.x->data),
            static_cast<uint32_t>(f.n), vectorized ? 1u : 0u, 1.0f / static_cast<float>(f.n), f.eps,
            f.offset);
    };
    switch (block_threads(f.n)) {
        case 128: return go(std::integral_constant<int, 4>{});
        case 256: return go(std::integral_constant<int, 8>{});
        case 512: return go(std::integral_constant<int, 16>{});
        default: return go(std::integral_constant<int, 32>{});
    }
}

// Dispatch over (mode, X, W, AFFINE) like ops.rs:136-184; `L` is a functor
// template invoked as L::template run<X, W, M, AFFINE>(args).
template <template <typename, typename, int, bool> class L, typename Args>
void dispatch(int mode, const kcr_tensor* x, const kcr_tensor* w, const Args& a) {
    auto with_mode = [&](auto xtag) {
        using X = decltype(xtag);
        auto go = [&](auto wtag, auto affine) {
            using W = decltype(wtag);
            constexpr bool AFF = decltype(affine)::value;
            switch (mode) {
                case MODE_LLAMA: L<X, W, MODE_LLAMA, AFF>::run(a); break;
                case MODE_GEMMA: L<X, W, MODE_GEMMA, AFF>::run(a); break;
                default: L<X, W, MODE_NONE, AFF>::run(a); break;
            }
        };
        if (!w) {
            go(X{}, std::false_type{});
        } else if (w->dtype == x->dtype) {
            go(X{}, std::true_type{});
        } else {
            go(float{}, std::true_type{});
        }
    };
    switch (x->dtype) {
        case KCR_FLOAT16: with_mode(f16_t{}); break;
        case KCR_BFLOAT16: with_mode(bf16_t{}); break;
        default: with_mode(float{}); break;
    }
}

template <typename X, typename W, int M, bool AFFINE>
struct FwdLaunch {
    static void run(const Fwd& f) {
        launch_fwd<X, W, M, AFFINE>(f);
        check_launch("launch rms_norm_fwd");
    }
};

struct Bwd {
    const kcr_tensor *dx, *dw_partial, *dy, *x, *w, *rstd;
    int64_t blocks, rows, n;
    float offset;
    hipStream_t stream;
};

template <typename X, typename W, int M, bool AFFINE>
struct BwdLaunch {
    static void run(const Bwd& b) {
        // Without dy the gradient is read from dx (in place).
        const void* dy = b.dy ? b.dy->data : b.dx->data;
        float* dwp = AFFINE ? static_cast<float*>(b.dw_partial->data) : nullptr;
        constexpr bool kWaveForm =
            vec_of<X>() == 8 && (!AFFINE || std::is_same<W, X>::value || std::is_same<W, float>::value);
        if constexpr (kWaveForm) {
            const bool aligned = aligned16(b.dx->data) && aligned16(dy) && aligned16(b.x->data) &&
                                 (!AFFINE || (aligned16(b.w->data) && aligned16(dwp)));
            const uint32_t nvec = static_cast<uint32_t>(b.n / 8);
            if (aligned && b.n % 8 == 0 && nvec <= 512 && b.blocks <= 0xffffffffll) {
                auto go = [&](auto chunks_tag) {
                    constexpr int CH = decltype(chunks_tag)::value;
                    const uint64_t grid = (static_cast<uint64_t>(b.blocks) + kWaves - 1) / kWaves;
                    rms_bwd_wave<X, W, M, AFFINE, CH><<<static_cast<unsigned>(grid), 64 * kWaves, 0, b.stream>>>(
                        static_cast<u32x4*>(b.dx->data), dwp, static_cast<const u32x4*>(dy),
                        static_cast<const u32x4*>(b.x->data),
                        static_cast<const u32x4*>(AFFINE ? b.w->data : b.x->data),
                        static_cast<const float*>(b.rstd->data), static_cast<uint32_t>(b.rows), nvec,
                        static_cast<uint32_t>(b.blocks), 1.0f / static_cast<float>(b.n), b.offset);
                };
                const uint32_t chunks = (nvec + 63) / 64;
                // Rows of 8 chunks: two waves per partial row (79.0 -> 71.3 us at
                // 16384 x 4096 bf16 with 1024 partial rows).
                if (chunks > 4) {
                    rms_bwd_split<X, W, M, AFFINE, 8><<<static_cast<unsigned>(b.blocks), 128, 0, b.stream>>>(
                        static_cast<u32x4*>(b.dx->data), dwp, static_cast<const u32x4*>(dy),
                        static_cast<const u32x4*>(b.x->data),
                        static_cast<const u32x4*>(AFFINE ? b.w->data : b.x->data),
                        static_cast<const float*>(b.rstd->data), static_cast<uint32_t>(b.rows), nvec,
                        static_cast<uint32_t>(b.blocks), 1.0f / static_cast<float>(b.n), b.offset);
                    check_launch("launch rms_norm_bwd");
                    return;
                }
                if (chunks <= 1) go(std::integral_constant<int, 1>{});
                else if (chunks <= 2) go(std::integral_constant<int, 2>{});
                else if (chunks <= 4) go(std::integral_constant<int, 4>{});
                else go(std::integral_constant<int, 8>{});
                check_launch("launch rms_norm_bwd");
                return;
            }
        }
        rms_bwd_block<X, W, M, AFFINE><<<static_cast<unsigned>(b.blocks), block_threads(b.n), 0, b.stream>>>(
            static_cast<X*>(b.dx->data), dwp, static_cast<const X*>(dy),
            static_cast<const X*>(b.x->data), static_cast<const W*>(AFFINE ? b.w->data : b.x->data),
            static_cast<const float*>(b.rstd->data), static_cast<uint32_t>(b.rows),
            static_cast<uint32_t>(b.n), 1.0f / static_cast<float>(b.n), b.offset);
        check_launch("launch rms_norm_bwd");
    }
};

}  // namespace
}  // namespace kcr

using namespace kcr;

extern "C" int kcr_rms_norm_forward(const kcr_tensor* y, const kcr_tensor* rstd,
                                    const kcr_tensor* x, const kcr_tensor* weight, double eps,
                                    double offset, const char* casting_mode, void* stream) {
    return guarded([&] {
        if (!y || !rstd || !x) throw value_error("y, rstd and x are required");
        const int mode = parse_mode(casting_mode);
        int64_t rows, n;
        rows_and_cols(x, rows, n);
        check_like(y, x, "y", "x");
        check_f32(rstd, rows, "rstd");
        check_weight(weight, n);
        if (rows == 0 || n == 0) return;
        check_input_dtype(x);
        check_weight_dtype(weight, x);
        check_contiguous(x, "x");
        check_contiguous(y, "y");
        check_contiguous(rstd, "rstd");
        check_contiguous(weight, "weight");
        Fwd f{y, rstd, x, weight, rows, n, static_cast<float>(eps), static_cast<float>(offset),
              static_cast<hipStream_t>(stream)};
        dispatch<FwdLaunch>(mode, x, weight, f);
    });
}

extern "C" int kcr_rms_norm_backward(const kcr_tensor* dx, const kcr_tensor* dw_partial,
                                     const kcr_tensor* dy, const kcr_tensor* x,
                                     const kcr_tensor* weight, const kcr_tensor* rstd,
                                     double offset, const char* casting_mode, void* stream) {
    return guarded([&] {
        if (!dx || !x || !rstd) throw value_error("dx, x and rstd are required");
        const int mode = parse_mode(casting_mode);
        int64_t rows, n;
        rows_and_cols(x, rows, n);
        check_like(dx, x, "dx", "x");
        if (dy) check_like(dy, x, "dy", "x");
        check_f32(rstd, rows, "rstd");
        check_weight(weight, n);
        if (n == 0) return;
        int64_t blocks;
        if (weight && dw_partial) {
            if (dw_partial->ndim != 2 || dw_partial->shape[1] != n || dw_partial->shape[0] < 1 ||
                dw_partial->shape[0] > kMaxGridX) {
                throw value_error("dw_partial must have shape [blocks, " + std::to_string(n) +
                                  "] with blocks > 0, got " + shape_string(*dw_partial));
            }
            blocks = dw_partial->shape[0];
            check_f32(dw_partial, blocks * n, "dw_partial");
        } else if (weight) {
            throw value_error("dw_partial is required with a weight");
        } else {
            if (rows == 0) return;
            blocks = rows;
        }
        check_input_dtype(x);
        check_weight_dtype(weight, x);
        check_contiguous(x, "x");
        check_contiguous(dx, "dx");
        check_contiguous(dy, "dy");
        check_contiguous(rstd, "rstd");
        check_contiguous(weight, "weight");
        if (weight) check_contiguous(dw_partial, "dw_partial");
        Bwd b{dx, weight ? dw_partial : nullptr, dy, x, weight, rstd, blocks, rows, n,
              static_cast<float>(offset), static_cast<hipStream_t>(stream)};
        dispatch<BwdLaunch>(mode, x, weight, b);
    });
}

extern "C" int kcr_rms_norm_reduce_weight_grad(const kcr_tensor* dw, const kcr_tensor* dw_partial,
                                               void* stream) {
    return guarded([&] {
        if (!dw || !dw_partial) throw value_error("dw and dw_partial are required");
        if (dw->ndim != 1) {
            throw value_error("dw must be one-dimensional, got shape " + shape_string(*dw));
        }
        const int64_t n = dw->shape[0];
        if (dw_partial->ndim != 2 || dw_partial->shape[1] != n ||
            dw_partial->shape[0] > 4294967295ll) {
            throw value_error("dw_partial must have shape [blocks, " + std::to_string(n) +
                              "], got " + shape_string(*dw_partial));
        }
        const int64_t blocks = dw_partial->shape[0];
        check_f32(dw_partial, blocks * n, "dw_partial");
        if (n == 0) return;
        check_contiguous(dw, "dw");
        check_contiguous(dw_partial, "dw_partial");
        auto s = static_cast<hipStream_t>(stream);
        const unsigned grid = static_cast<unsigned>((n + kReduceCols - 1) / kReduceCols);
        constexpr unsigned threads = 64 * kReduceWaves;
        const auto* p = static_cast<const float*>(dw_partial->data);
        switch (dw->dtype) {
            case KCR_FLOAT16:
                reduce_weight_grad<f16_t><<<grid, threads, 0, s>>>(static_cast<f16_t*>(dw->data), p,
                                                               blocks, n);
                break;
            case KCR_BFLOAT16:
                reduce_weight_grad<bf16_t><<<grid, threads, 0, s>>>(static_cast<bf16_t*>(dw->data), p,
                                                                blocks, n);
                break;
            case KCR_FLOAT32:
                reduce_weight_grad<float><<<grid, threads, 0, s>>>(static_cast<float*>(dw->data), p,
                                                               blocks, n);
                break;
            default:
                throw value_error("unsupported dtype for dw, expected float16, bfloat16 or float32");
        }
        check_launch("launch reduce_weight_grad");
    });
}
