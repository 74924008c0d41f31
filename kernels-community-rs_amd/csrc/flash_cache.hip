// KV-cache append with rotary embedding, the first half of
// flash_attn_with_kvcache (flash-attn2-rs/src/host/cache/mod.rs:36-320 and the
// kernel of src/device/cache.rs:26-330).
//
// New key/value row r of batch b goes to cache position lengths[b] + r: row
// `position` of cache batch cache_batch_idx[b] (or b), or row position % page of
// page block_table[b, position / page]. Positions past the capacity (or the
// rotary table) and invalid batch / page indices are skipped, as in the
// reference. With rotary tables (cos/sin [positions, rotary_dim / 2]), K is
// rotated at its position and Q at lengths[b] + (advance_q ? r : 0); columns
// d < rotary_dim pair up as (d, d ^ 1) (interleaved) or (d, d +- rotary_dim / 2)
// and take angle position * rotary_dim / 2 + frequency:
//   out = x_d * cos + x_partner * (first of the pair ? -sin : sin)
// computed in fp32 and rounded to the element type.
//
// MI355X shape: one lane per 16-byte vector (8 columns) of a row; the rotary
// partner vector is one more 16-byte load (the same vector when interleaved).
// The op moves a few rows per sequence, so it is launch-bound, not HBM-bound.
// Caches or sources with rows that are not 16-byte aligned (odd strides, views
// into shared storage) take a one-element-per-lane kernel.

#include "attention.h"

namespace kcr {
namespace attn {

struct CacheUpdateParams {
    const uint16_t* k;   // new keys [B, Snew, Hk, D]
    const uint16_t* v;
    uint16_t* kc;        // caches [batches | pages, rows, Hk, D]
    uint16_t* vc;
    const uint16_t* q;   // [B, Sq, H, D], rotated into q_out when rotary_dim > 0
    uint16_t* q_out;
    const uint16_t* cos;
    const uint16_t* sin;
    const int32_t* lengths;
    const int32_t* cache_idx;
    const int32_t* table;
    int64_t k_b, k_s, k_h, v_b, v_s, v_h;
    int64_t kc_b, kc_s, kc_h, vc_b, vc_s, vc_h;
    int64_t q_b, q_s, q_h, qo_b, qo_s, qo_h;
    int64_t table_stride;
    int32_t batch, snew, hk, sq, hq, d;
    int32_t capacity, cache_batches, page_size, table_cols;
    int32_t rotary_dim, rotary_rows, interleaved, advance_q;
    int64_t kv_vectors, q_vectors;  // work items: B * Snew * Hk * D / 8, B * Sq * H * D / 8
};

template <typename T>
__device__ __forceinline__ float elem_to_f32(uint16_t x) {
    if constexpr (std::is_same<T, bf16_t>::value) return bf16_bits_to_f32(x);
    return f16_bits_to_f32(x);
}
template <typename T>
__device__ __forceinline__ uint16_t f32_to_elem(float x) {
    if constexpr (std::is_same<T, bf16_t>::value) return static_cast<uint16_t>(f32_to_bf16_bits(x));
    return static_cast<uint16_t>(f32_to_f16_bits(x));
}

// Rotates the 8 columns c0 .. c0 + 7 of `row` (rotary columns only) at `position`.
template <typename T>
__device__ __forceinline__ u32x4 rotate8(const uint16_t* row, int c0, const CacheUpdateParams& p,
                                         uint32_t position) {
    const u32x4 raw = *reinterpret_cast<const u32x4*>(row + c0);
    if (c0 >= p.rotary_dim) return raw;
    const int half = p.rotary_dim / 2;
    uint16_t x[8], y[8];
    __builtin_memcpy(x, &raw, 16);
    if (p.interleaved) {
        __builtin_memcpy(y, &raw, 16);
    } else {
        const int pc = c0 < half ? c0 + half : c0 - half;
        const u32x4 pr = *reinterpret_cast<const u32x4*>(row + pc);
        __builtin_memcpy(y, &pr, 16);
    }
    const uint16_t* cs = p.cos + static_cast<int64_t>(position) * half;
    const uint16_t* sn = p.sin + static_cast<int64_t>(position) * half;
    uint16_t r[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int d = c0 + e;
        bool first;
        float other;
        int freq;
        if (p.interleaved) {
            first = (d & 1) == 0;
            other = elem_to_f32<T>(y[e ^ 1]);
            freq = d / 2;
        } else {
            first = d < half;
            other = elem_to_f32<T>(y[e]);
            freq = d % half;
        }
        const float a = elem_to_f32<T>(x[e]);
        const float c = elem_to_f32<T>(cs[freq]);
        const float s = elem_to_f32<T>(sn[freq]);
        // Two rounded products and a rounded sum (no fused multiply-add), as the
        // reference evaluates a * c + b * (+-s).
        r[e] = f32_to_elem<T>(__fadd_rn(__fmul_rn(a, c), __fmul_rn(other, first ? -s : s)));
    }
    u32x4 out;
    __builtin_memcpy(&out, r, 16);
    return out;
}

template <typename T>
__global__ void __launch_bounds__(256) cache_update_kernel(const CacheUpdateParams p) {
    const int vpr = p.d / 8;  // vectors per row
    const int64_t total = p.kv_vectors + p.q_vectors;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        if (i < p.kv_vectors) {
            const int c0 = static_cast<int>(i % vpr) * 8;
            int64_t t = i / vpr;
            const int h = static_cast<int>(t % p.hk);
            t /= p.hk;
            const int r = static_cast<int>(t % p.snew);
            const int b = static_cast<int>(t / p.snew);
            const int start = p.lengths[b];
            const int64_t position = static_cast<int64_t>(start) + r;
            if (start < 0 || position >= p.capacity || (p.rotary_dim > 0 && position >= p.rotary_rows)) continue;
            int64_t cb, crow;
            if (p.table) {
                const int64_t col = position / p.page_size;
                if (col >= p.table_cols) continue;
                const int page = p.table[b * p.table_stride + col];
                if (page < 0 || page >= p.cache_batches) continue;
                cb = page;
                crow = position % p.page_size;
            } else {
                const int idx = p.cache_idx ? p.cache_idx[b] : b;
                if (idx < 0 || idx >= p.cache_batches) continue;
                cb = idx;
                crow = position;
            }
            const uint16_t* krow = p.k + b * p.k_b + r * p.k_s + h * p.k_h;
            const uint16_t* vrow = p.v + b * p.v_b + r * p.v_s + h * p.v_h;
            const u32x4 kval = p.rotary_dim > 0 ? rotate8<T>(krow, c0, p, static_cast<uint32_t>(position))
                                                : *reinterpret_cast<const u32x4*>(krow + c0);
            *reinterpret_cast<u32x4*>(p.kc + cb * p.kc_b + crow * p.kc_s + h * p.kc_h + c0) = kval;
            *reinterpret_cast<u32x4*>(p.vc + cb * p.vc_b + crow * p.vc_s + h * p.vc_h + c0) =
                *reinterpret_cast<const u32x4*>(vrow + c0);
        } else {
            const int64_t j = i - p.kv_vectors;
            const int c0 = static_cast<int>(j % vpr) * 8;
            int64_t t = j / vpr;
            const int h = static_cast<int>(t % p.hq);
            t /= p.hq;
            const int r = static_cast<int>(t % p.sq);
            const int b = static_cast<int>(t / p.sq);
            const uint16_t* qrow = p.q + b * p.q_b + r * p.q_s + h * p.q_h;
            uint16_t* orow = p.q_out + b * p.qo_b + r * p.qo_s + h * p.qo_h;
            const int start = p.lengths[b];
            const int64_t position = static_cast<int64_t>(start) + (p.advance_q ? r : 0);
            // Rows whose position has no rotary entry keep their values.
            const bool rot = start >= 0 && position < p.rotary_rows;
            *reinterpret_cast<u32x4*>(orow + c0) = rot ? rotate8<T>(qrow, c0, p, static_cast<uint32_t>(position))
                                                       : *reinterpret_cast<const u32x4*>(qrow + c0);
        }
    }
}

// Caches or sources whose rows are not 16-byte aligned: one lane per element,
// the same positions, skips and rotary arithmetic.
template <typename T>
__global__ void __launch_bounds__(256) cache_update_scalar_kernel(const CacheUpdateParams p) {
    const int64_t kv_elems = p.kv_vectors * 8, q_elems = p.q_vectors * 8;
    const int half = p.rotary_dim / 2;
    auto rot = [&](const uint16_t* row, int dcol, uint32_t position) -> uint16_t {
        if (dcol >= p.rotary_dim) return row[dcol];
        bool first;
        int other, freq;
        if (p.interleaved) {
            first = (dcol & 1) == 0;
            other = dcol ^ 1;
            freq = dcol / 2;
        } else {
            first = dcol < half;
            other = first ? dcol + half : dcol - half;
            freq = dcol % half;
        }
        const float a = elem_to_f32<T>(row[dcol]);
        const float b = elem_to_f32<T>(row[other]);
        const float c = elem_to_f32<T>(p.cos[static_cast<int64_t>(position) * half + freq]);
        const float sn = elem_to_f32<T>(p.sin[static_cast<int64_t>(position) * half + freq]);
        return f32_to_elem<T>(__fadd_rn(__fmul_rn(a, c), __fmul_rn(b, first ? -sn : sn)));
    };
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < kv_elems + q_elems;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        if (i < kv_elems) {
            const int dcol = static_cast<int>(i % p.d);
            int64_t t = i / p.d;
            const int h = static_cast<int>(t % p.hk);
            t /= p.hk;
            const int r = static_cast<int>(t % p.snew);
            const int b = static_cast<int>(t / p.snew);
            const int start = p.lengths[b];
            const int64_t position = static_cast<int64_t>(start) + r;
            if (start < 0 || position >= p.capacity || (p.rotary_dim > 0 && position >= p.rotary_rows)) continue;
            int64_t cb, crow;
            if (p.table) {
                const int64_t col = position / p.page_size;
                if (col >= p.table_cols) continue;
                const int page = p.table[b * p.table_stride + col];
                if (page < 0 || page >= p.cache_batches) continue;
                cb = page;
                crow = position % p.page_size;
            } else {
                const int idx = p.cache_idx ? p.cache_idx[b] : b;
                if (idx < 0 || idx >= p.cache_batches) continue;
                cb = idx;
                crow = position;
            }
            const uint16_t* krow = p.k + b * p.k_b + r * p.k_s + h * p.k_h;
            const uint16_t* vrow = p.v + b * p.v_b + r * p.v_s + h * p.v_h;
            p.kc[cb * p.kc_b + crow * p.kc_s + h * p.kc_h + dcol] =
                p.rotary_dim > 0 ? rot(krow, dcol, static_cast<uint32_t>(position)) : krow[dcol];
            p.vc[cb * p.vc_b + crow * p.vc_s + h * p.vc_h + dcol] = vrow[dcol];
        } else {
            const int64_t j = i - kv_elems;
            const int dcol = static_cast<int>(j % p.d);
            int64_t t = j / p.d;
            const int h = static_cast<int>(t % p.hq);
            t /= p.hq;
            const int r = static_cast<int>(t % p.sq);
            const int b = static_cast<int>(t / p.sq);
            const uint16_t* qrow = p.q + b * p.q_b + r * p.q_s + h * p.q_h;
            const int start = p.lengths[b];
            const int64_t position = static_cast<int64_t>(start) + (p.advance_q ? r : 0);
            const bool rotate = start >= 0 && position < p.rotary_rows;
            p.q_out[b * p.qo_b + r * p.qo_s + h * p.qo_h + dcol] =
                rotate ? rot(qrow, dcol, static_cast<uint32_t>(position)) : qrow[dcol];
        }
    }
}

}  // namespace attn
}  // namespace kcr

using namespace kcr;
using namespace kcr::attn;

extern "C" int kcr_flash_cache_update(const kcr_tensor* q, const kcr_tensor* kcache, const kcr_tensor* vcache,
                                      const kcr_tensor* k, const kcr_tensor* v, const kcr_tensor* seqlens,
                                      const kcr_tensor* rotary_cos, const kcr_tensor* rotary_sin,
                                      const kcr_tensor* cache_batch_idx, const kcr_tensor* block_table,
                                      int interleaved, int advance_q, const kcr_tensor* q_out, void* stream) {
    return guarded([&] {
        for (auto [t, name] : {std::pair{q, "q"}, {kcache, "kcache"}, {vcache, "vcache"}, {k, "k"}, {v, "v"}}) {
            check_qkv(t, name, 4);
            if (t->dtype != q->dtype) throw type_error("cache update requires one FP16/BF16 dtype");
            require_device(t, name);
        }
        const int64_t B = q->shape[0], Sq = q->shape[1], H = q->shape[2], D = q->shape[3];
        const int64_t Bc = kcache->shape[0], S = kcache->shape[1], Hk = kcache->shape[2];
        if (shape_of(*kcache) != shape_of(*vcache) || shape_of(*k) != shape_of(*v) || k->shape[0] != B ||
            k->shape[2] != Hk || k->shape[3] != D || kcache->shape[3] != D || Hk <= 0 || H % Hk != 0 ||
            D % 8 != 0 || D > 256) {
            throw value_error("inconsistent cache update shapes");
        }
        auto meta = [&](const kcr_tensor* t, const char* name, int ndim) {
            if (!t) return;
            if (t->dtype != KCR_INT32 || t->ndim != ndim || t->shape[0] != B || t->strides[ndim - 1] != 1) {
                throw value_error(std::string(name) + " must be int32 with batch rows and unit last stride");
            }
            require_device(t, name);
        };
        if (!seqlens) throw value_error("cache lengths are required when appending K/V");
        meta(seqlens, "lengths", 1);
        meta(cache_batch_idx, "indices", 1);
        meta(block_table, "block_table", 2);
        if (block_table && (cache_batch_idx || S % 256 != 0)) throw value_error("invalid paged cache metadata");
        const int64_t capacity = block_table ? S * block_table->shape[1] : S;
        if (!block_table && !cache_batch_idx && Bc < B) throw value_error("cache batch must cover Q without indices");
        if (capacity > INT32_MAX || Bc > INT32_MAX) throw value_error("cache dimensions must fit int32");
        int64_t rd = 0, rows = 0;
        if ((rotary_cos != nullptr) != (rotary_sin != nullptr)) {
            throw value_error("cos and sin must be supplied together");
        }
        if (rotary_cos) {
            if (rotary_cos->ndim != 2 || shape_of(*rotary_cos) != shape_of(*rotary_sin) ||
                rotary_cos->dtype != q->dtype || rotary_sin->dtype != q->dtype || !is_contiguous(*rotary_cos) ||
                !is_contiguous(*rotary_sin)) {
                throw value_error("rotary tables must be contiguous [positions,rotary_dim/2] in Q dtype/device");
            }
            require_device(rotary_cos, "rotary_cos");
            require_device(rotary_sin, "rotary_sin");
            rd = rotary_cos->shape[1] * 2;
            rows = rotary_cos->shape[0];
            if (rd > D || rd % 16 != 0 || rows < capacity || rows > INT32_MAX) {
                throw value_error(
                    "rotary dimension must be divisible by 16 and fit D; positions must cover cache capacity");
            }
            if (!q_out || shape_of(*q_out) != shape_of(*q) || q_out->dtype != q->dtype || q_out->strides[3] != 1) {
                throw value_error("q_out must match q when rotary tables are given");
            }
            require_device(q_out, "q_out");
        }
        CacheUpdateParams p{};
        p.k = static_cast<const uint16_t*>(k->data);
        p.v = static_cast<const uint16_t*>(v->data);
        p.kc = static_cast<uint16_t*>(kcache->data);
        p.vc = static_cast<uint16_t*>(vcache->data);
        p.q = static_cast<const uint16_t*>(q->data);
        p.q_out = rd > 0 ? static_cast<uint16_t*>(q_out->data) : nullptr;
        p.cos = rd > 0 ? static_cast<const uint16_t*>(rotary_cos->data) : nullptr;
        p.sin = rd > 0 ? static_cast<const uint16_t*>(rotary_sin->data) : nullptr;
        p.lengths = static_cast<const int32_t*>(seqlens->data);
        p.cache_idx = cache_batch_idx ? static_cast<const int32_t*>(cache_batch_idx->data) : nullptr;
        p.table = block_table ? static_cast<const int32_t*>(block_table->data) : nullptr;
        p.k_b = k->strides[0]; p.k_s = k->strides[1]; p.k_h = k->strides[2];
        p.v_b = v->strides[0]; p.v_s = v->strides[1]; p.v_h = v->strides[2];
        p.kc_b = kcache->strides[0]; p.kc_s = kcache->strides[1]; p.kc_h = kcache->strides[2];
        p.vc_b = vcache->strides[0]; p.vc_s = vcache->strides[1]; p.vc_h = vcache->strides[2];
        p.q_b = q->strides[0]; p.q_s = q->strides[1]; p.q_h = q->strides[2];
        if (rd > 0) { p.qo_b = q_out->strides[0]; p.qo_s = q_out->strides[1]; p.qo_h = q_out->strides[2]; }
        p.table_stride = block_table ? block_table->strides[0] : 0;
        p.batch = static_cast<int32_t>(B);
        p.snew = static_cast<int32_t>(k->shape[1]);
        p.hk = static_cast<int32_t>(Hk);
        p.sq = static_cast<int32_t>(Sq);
        p.hq = static_cast<int32_t>(H);
        p.d = static_cast<int32_t>(D);
        p.capacity = static_cast<int32_t>(capacity);
        p.cache_batches = static_cast<int32_t>(Bc);
        p.page_size = static_cast<int32_t>(S);
        p.table_cols = block_table ? static_cast<int32_t>(block_table->shape[1]) : 0;
        p.rotary_dim = static_cast<int32_t>(rd);
        p.rotary_rows = static_cast<int32_t>(rows);
        p.interleaved = interleaved ? 1 : 0;
        p.advance_q = advance_q ? 1 : 0;
        // Work items in 8-column vectors (the scalar kernel walks 8 x as many).
        if (D % 8 != 0) throw value_error("head size must be a multiple of 8 (pad the caches)");
        p.kv_vectors = B * k->shape[1] * Hk * (D / 8);
        p.q_vectors = rd > 0 ? B * Sq * H * (D / 8) : 0;
        const int64_t total = p.kv_vectors + p.q_vectors;
        if (total == 0) return;
        auto s = static_cast<hipStream_t>(stream);
        // 16-byte vectors need D % 8 == 0 and 16-byte aligned rows everywhere.
        bool vec = D % 8 == 0;
        for (auto* t : {q, kcache, vcache, k, v}) vec = vec && rows_aligned16(t);
        if (rd > 0) vec = vec && rows_aligned16(q_out);
        if (vec) {
            const unsigned grid = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 65536));
            if (q->dtype == KCR_BFLOAT16) {
                cache_update_kernel<bf16_t><<<grid, 256, 0, s>>>(p);
            } else {
                cache_update_kernel<f16_t><<<grid, 256, 0, s>>>(p);
            }
        } else {
            const unsigned grid = static_cast<unsigned>(std::min<int64_t>((total * 8 + 255) / 256, 65536));
            if (q->dtype == KCR_BFLOAT16) {
                cache_update_scalar_kernel<bf16_t><<<grid, 256, 0, s>>>(p);
            } else {
                cache_update_scalar_kernel<f16_t><<<grid, 256, 0, s>>>(p);
            }
        }
        check_launch("launch cache_update");
    });
}
