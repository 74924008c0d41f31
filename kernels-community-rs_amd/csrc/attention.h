// Shared pieces of the FlashAttention-2 kernels (forward and backward):
// MFMA operand types, the launch parameters, score/mask math and the host-side
// argument normalisation of flash-attn2-rs/src/host/forward/mod.rs:303-328.
#pragma once

#include "common.h"

#include <initializer_list>

namespace kcr {
namespace attn {

// ---------------------------------------------------------------------------
// MFMA 32x32x16 (gfx950). Operand layout (verified on the device):
//   A (32 x 16): lane l holds A[l % 32][8 * (l / 32) + j], j = 0..7
//   B (16 x 32): lane l holds B[8 * (l / 32) + j][l % 32]
//   C (32 x 32): lane l, register r holds C[8 * (r / 4) + 4 * (l / 32) + r % 4][l % 32]
// ---------------------------------------------------------------------------
using bf16x8 = __bf16 __attribute__((ext_vector_type(8)));
using f16x8 = _Float16 __attribute__((ext_vector_type(8)));
using f32x16 = float __attribute__((ext_vector_type(16)));

template <typename T>
__device__ __forceinline__ f32x16 mfma32(const u32x4& a, const u32x4& b, const f32x16& c) {
    if constexpr (sizeof(T) == 2 && std::is_same<T, bf16_t>::value) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                        __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                       __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
}

using bf16x2 = __bf16 __attribute__((ext_vector_type(2)));
using f16x2 = _Float16 __attribute__((ext_vector_type(2)));
using f32x2 = float __attribute__((ext_vector_type(2)));

// Packs two f32 into the element type T (round to nearest even), lo in the low
// half: one v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32 on gfx950.
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    const f32x2 v = {lo, hi};
    if constexpr (std::is_same<T, bf16_t>::value) {
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
    } else {
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
    }
}

// Maximum of the 32 scores one lane holds (two 16-register halves) as a chain of
// 16 v_maximum3_f32. IEEE maximum propagates NaN, which the row's output would
// carry anyway; fmaxf would first quieten every operand (one extra v_max each).
__device__ __forceinline__ float max3f(float a, float b, float c) {
    return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}
__device__ __forceinline__ float lane_max32(const f32x16& a, const f32x16& b) {
    float m0 = max3f(a[0], a[1], a[2]);
    float m1 = max3f(b[0], b[1], b[2]);
#pragma unroll
    for (int r = 3; r < 15; r += 2) {
        m0 = max3f(m0, a[r], a[r + 1]);
        m1 = max3f(m1, b[r], b[r + 1]);
    }
    return max3f(m0, m1, __builtin_elementwise_maximum(a[15], b[15]));
}

// Buffer resource over `bytes` bytes at `base`: loads at offsets >= bytes return 0
// (hardware range check), which zero-fills the tile rows past the sequence end.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), 0x00020000);
}

__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, 0));
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

constexpr float kLog2e = 1.4426950408889634f;

// tanh(y) from one exp2 and one reciprocal, 1 - 2 / (e^(2|y|) + 1) with the
// sign of y (absolute error ~1e-7; e^(2|y|) = inf gives 1). The tiled softcap
// paths use it: libm's tanhf inlined per score is several times the VALU work
// and registers.
__device__ __forceinline__ float tanh_exp2(float y) {
    const float e = fast_exp2((2.0f * kLog2e) * fabsf(y));
    return copysignf(1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f), y);
}
constexpr float kLn2 = 0.6931471805599453f;

// Launch parameters shared by the dense and varlen forward kernels. Strides are
// in elements. Window bounds follow the normalisation of the reference
// (host/forward/mod.rs:310-328): -1 = unbounded on that side.
struct FwdParams {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* lse;
    const float* alibi;
    const int32_t* cu_q;
    const int32_t* cu_k;
    const int32_t* seqused_k;
    const int32_t* leftpad_k;
    int64_t q_b, q_s, q_h;
    int64_t k_b, k_s, k_h;
    int64_t v_b, v_s, v_h;
    int64_t o_b, o_s, o_h;
    int64_t lse_b, lse_h;  // dense: [B,H,Sq] -> H*Sq, Sq; varlen: [H,Tq] -> 0, Tq
    int32_t total_q, total_k;    // varlen: rows of q and k (bounds for cu_seqlens)
    int32_t batch, heads, kv_heads, gqa;
    int32_t seqlen_q, seqlen_k;  // dense sizes; varlen: max_seqlen_q / max_seqlen_k
    int32_t head_dim;            // real head size (<= bucket D)
    int32_t window_left, window_right;
    int32_t q_blocks;            // query tiles per (batch, head)
    int32_t xcd_groups;          // 1: group the query heads of one KV head on one XCD
    int32_t seq_major;           // 1: sequence-major block order (tiled kernel)
    int32_t alibi_b;             // alibi batch stride (0 for [H])
    int32_t alibi_causal;
    const int64_t* rng_state;    // dropout: device [seed, offset], or null (use the fields below)
    uint64_t drop_seed, drop_offset;
    uint32_t drop_threshold;     // keep when byte <= threshold; 255 = no dropout
    float inv_keep;              // 1 / (1 - p)
    float scale_log2;            // softmax scale * log2(e), no softcap
    float tanh_scale;            // softcap: tanh(raw * tanh_scale) * scale_eff
    float scale_eff_log2;        // softcap: softcap * sign(scale) * log2(e)
    // KV-cache mode (varlen kernels; flash-attn2-rs/src/device/varlen/mod.rs:60-170
    // with CACHED): the keys of sequence b are rows [leftpad_k[b], seqused_k[b])
    // of cache batch cache_idx[b] (or b), or of the pages block_table[b, :].
    int32_t cache_mode;
    int32_t capacity;            // rows per cache batch (or table_cols * page_size)
    int32_t cache_batches;       // cache batches (or pages)
    const int32_t* cache_idx;
    const int32_t* block_table;  // paged K/V: [batch, table_cols] page indices
    int64_t table_stride;
    int32_t table_cols;
    int32_t page_size;           // rows per page, a multiple of the 64-row tile
    int64_t k_page, v_page;      // element strides between pages
    // Split-KV (tiled varlen kernel): n_splits > 1 writes per-split fp32 partials
    // o_part [n_splits, H, Tq, D] (normalised) and lse_part [n_splits, H, Tq].
    int32_t n_splits;
    int32_t scored;              // tiled kernels: softcap and / or ALiBi score transform
    float* o_part;
    float* lse_part;
    // Batched cache queries: rows_per_seq > 0 means q/o [B, rows_per_seq, H, D]
    // and lse [B, H, rows_per_seq] addressed through q_b / o_b / lse_b, with no
    // cu_q; sequence b's rows are packed rows b * rows_per_seq .. for the
    // split partials. 0: packed rows through cu_q (q_b = o_b = lse_b = 0).
    int32_t rows_per_seq;
    // Added to every seqused_k entry (cache mode: the appended rows).
    int32_t seqused_add;
};

// Packed-sequence bounds of sequence b (device/varlen/mod.rs:79-136): query rows
// [qs, qs + sq) of the packed q, keys from row k_row0 of K batch k_batch (cache
// mode) or of the packed K. Metadata is trusted as in the reference; only memory
// bounds are guarded (ok = false: the block writes nothing).
struct VarSeq {
    int sq, sk, qs;
    int64_t k_row0, k_batch;
    bool ok;
};

__device__ __forceinline__ VarSeq varlen_seq(const FwdParams& p, int b) {
    VarSeq r{};
    const int qs = p.rows_per_seq ? b * p.rows_per_seq : p.cu_q[b];
    const int qe = p.rows_per_seq ? qs + p.rows_per_seq : p.cu_q[b + 1];
    int ks = 0, ke = p.capacity;
    int64_t kbatch = 0;
    if (p.cache_mode) {
        if (!p.block_table) {
            kbatch = p.cache_idx ? p.cache_idx[b] : b;
            if (kbatch < 0 || kbatch >= p.cache_batches) return r;
        }
    } else {
        ks = p.cu_k[b];
        ke = p.cu_k[b + 1];
    }
    const int len = p.seqused_k ? p.seqused_k[b] + p.seqused_add : ke - ks;
    const int pad = p.leftpad_k ? p.leftpad_k[b] : 0;
    if (qs < 0 || qe < qs || qe > p.total_q || ks < 0 || ke < ks || (!p.cache_mode && ke > p.total_k) ||
        pad < 0 || len < pad || len > ke - ks || qe - qs > p.seqlen_q) {
        return r;
    }
    r.sq = qe - qs;
    r.sk = len - pad;
    r.qs = qs;
    r.k_row0 = static_cast<int64_t>(ks + pad);
    r.k_batch = kbatch;
    r.ok = true;
    return r;
}

// Paged K/V: the page of the block table that holds key row kb of sequence b
// (tiles never cross pages: pages are multiples of the tile). Returns -1 for
// entries outside the table or the cache; such tiles read as zero.
__device__ __forceinline__ int64_t page_of(const FwdParams& p, int b, int kb) {
    const int col = kb / p.page_size;
    if (col >= p.table_cols) return -1;
    const int page = p.block_table[static_cast<int64_t>(b) * p.table_stride + col];
    return (page >= 0 && page < p.cache_batches) ? page : -1;
}

// Host-side normalisation of the attention options shared by all entry points.
struct Options {
    float scale;
    float tanh_scale;
    float scale_eff;
    int32_t window_left;
    int32_t window_right;
    int32_t alibi_causal;
};

// flash-attn2-rs/src/host/forward/mod.rs:303-328 (and varlen/mod.rs:250-268 with
// seqlen_k = max_seqlen_k).
inline Options normalize_options(int has_scale, double scale, int causal, int64_t wl, int64_t wr,
                                 double softcap, int64_t head_dim, int64_t seqlen_k) {
    if (wl < INT32_MIN || wl > INT32_MAX || wr < INT32_MIN || wr > INT32_MAX) {
        throw value_error("window sizes must fit int32");
    }
    Options o;
    const double s = has_scale ? scale : 1.0 / std::sqrt(static_cast<double>(head_dim));
    if (softcap > 0.0 && s != 0.0) {
        o.scale = static_cast<float>(std::copysign(softcap, s));
        o.tanh_scale = static_cast<float>(std::fabs(s) / softcap);
        o.scale_eff = o.scale;
    } else {
        o.scale = static_cast<float>(s);
        o.tanh_scale = 0.0f;
        o.scale_eff = static_cast<float>(s);
    }
    if (wl >= seqlen_k) wl = -1;
    if (wr >= seqlen_k) wr = -1;
    if (causal) wr = 0;
    o.alibi_causal = (wl < 0 && wr == 0) ? 1 : 0;
    if (wl < 0 && wr >= 0) wl = seqlen_k;
    if (wl >= 0 && wr < 0) wr = seqlen_k;
    o.window_left = static_cast<int32_t>(wl);
    o.window_right = static_cast<int32_t>(wr);
    return o;
}

// Dropout arguments (flash-attn2-rs/src/host/forward/mod.rs:73-131, 199): keep =
// 1 - p in f32, threshold = floor(keep * 255) in f32, 255 = no dropout.
struct DropoutArgs {
    uint32_t threshold = 255;
    float keep = 1.0f;
    float inv_keep = 1.0f;
    uint64_t seed = 0, offset = 0;
    const int64_t* state = nullptr;
};

inline DropoutArgs parse_dropout(const kcr_dropout* d, double softcap, const kcr_tensor* q) {
    DropoutArgs a;
    if (!d) return a;
    const double p = d->p;
    if (!std::isfinite(p) || p < 0.0 || p >= 1.0 || static_cast<float>(p) >= 1.0f) {
        throw value_error("p_dropout must be finite and in [0, 1) as float32");
    }
    if (!(static_cast<float>(p) > 0.0f)) return a;
    if (softcap > 0.0) throw value_error("softcap with dropout is not supported by FlashAttention v2");
    a.keep = 1.0f - static_cast<float>(p);
    a.threshold = static_cast<uint32_t>(a.keep * 255.0f);
    a.inv_keep = 1.0f / a.keep;
    if (d->rng_state) {
        const kcr_tensor* t = d->rng_state;
        if (t->dtype != KCR_INT64 || t->ndim != 1 || t->shape[0] != 2 || (t->strides[0] != 1) ||
            t->device < 0 || t->device != q->device || reinterpret_cast<uintptr_t>(t->data) % 8 != 0) {
            throw value_error("rng_state must be a contiguous CUDA int64 tensor of shape [2] on q's device");
        }
        if (d->offset != 0) throw value_error("offset must be zero when seed is an RNG-state tensor");
        a.state = static_cast<const int64_t*>(t->data);
    } else {
        a.seed = d->seed;
        a.offset = d->offset;
    }
    return a;
}

template <typename P>
inline void set_dropout(P& prm, const DropoutArgs& a) {
    prm.rng_state = a.state;
    prm.drop_seed = a.seed;
    prm.drop_offset = a.offset;
    prm.drop_threshold = a.threshold;
    prm.inv_keep = a.inv_keep;
}

inline const char* dtype_name(int dtype) {
    switch (dtype) {
        case KCR_FLOAT16: return "float16";
        case KCR_BFLOAT16: return "bfloat16";
        case KCR_FLOAT32: return "float32";
        default: return "other";
    }
}

// Common tensor checks for q/k/v-like tensors: half precision, unit last stride,
// 16-byte aligned rows (the kernels move 16-byte vectors).
inline void check_qkv(const kcr_tensor* t, const char* name, int ndim) {
    if (!t) throw value_error(std::string(name) + " is required");
    if (t->ndim != ndim) {
        throw value_error(std::string(name) + " must have " + std::to_string(ndim) +
                          " dimensions, got shape " + shape_string(*t));
    }
    if (t->dtype != KCR_FLOAT16 && t->dtype != KCR_BFLOAT16) {
        throw type_error(std::string(name) + " must be float16 or bfloat16, got " +
                         dtype_name(t->dtype));
    }
    if (t->strides[ndim - 1] != 1 && t->shape[ndim - 1] > 1) {
        throw value_error(std::string(name) + " must have a contiguous last dimension");
    }
}

inline bool rows_aligned16(const kcr_tensor* t) {
    if (!aligned16(t->data)) return false;
    for (int i = 0; i + 1 < t->ndim; ++i) {
        if (t->shape[i] > 1 && (t->strides[i] % 8) != 0) return false;
    }
    return true;
}

// XOR swizzle of the 16-byte chunks of a row-major LDS tile row with CH = 32
// (D = 256, 512-byte rows), CH = 16 (D = 128, 256-byte rows) or CH = 8 (D = 64,
// 128-byte rows): the chunk of row r is stored at chunk ^ kv_swizzle(r). Chosen for gfx950's 256-byte LDS
// bank window (measured on the device):
//   - ds_read_b128 serves 16 lanes per pass; they read 16 consecutive rows at one
//     logical chunk, and the swizzle maps those rows to 16 distinct 16-byte slots;
//   - ds_read_b64_tr_b16 serves 32 lanes per pass; they read 4 rows x 4 chunks,
//     and the swizzle gives each of the 4 rows its own 64-byte quarter.
// The value depends on row bits 0..3 only, so row offsets that are multiples of
// 16 keep it. A 512-byte row spans the bank window twice, so every row starts
// at bank 0 as with CH = 16; the CH = 16 values (< 16) then place the chunks
// in the same banks, and leave chunk bit 4 (which half of the row) unchanged.
template <int CH>
__device__ __forceinline__ int kv_swizzle(int row) {
    static_assert(CH == 8 || CH == 16 || CH == 32, "16-byte chunks per row: 8, 16 or 32");
    if constexpr (CH >= 16) {
        return 4 * (row & 3) + ((row >> 2) & 3);
    } else {
        return 4 * ((row >> 1) & 1) + ((row >> 2) & 1);
    }
}

using s16x4 = short __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16: inside each group of 16 lanes, lane L supplies the
// address of 4 consecutive 16-bit values; lane i receives value i % 4 of lanes
// i / 4, 4 + i / 4, 8 + i / 4 and 12 + i / 4 (a 4 x 16 -> 16 x 4 transpose).
__device__ __forceinline__ uint2 ds_read_tr16(const uint16_t* p) {
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(p));
    return __builtin_bit_cast(uint2, v);
}

// s_waitcnt vmcnt(0) (gfx9 encoding: expcnt / lgkmcnt left at their maximum);
// the direct LDS copies are tracked by vmcnt.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Compile-time loop: f(std::integral_constant<int, I>) for I = B .. E - 1.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// Direct HBM -> LDS copy issued from inline assembly: 16 bytes per lane from the
// buffer `rsrc` (descriptor words) at `voffset` into LDS at `lds_base` + 16 * lane.
// The compiler does not see these copies, so it inserts no wait for them before
// later LDS reads; the caller orders them with explicit vmcnt waits and barriers.
// NT sets the non-temporal cache policy, for data that no other block reads
// again (measured on MI355X: a decode K/V stream runs at ~6.8 TB/s with it and
// ~5.5 TB/s without).
template <bool NT = false>
__device__ __forceinline__ void dma_lds16(const u32x4& rsrc, uint32_t lds_base, uint32_t voffset) {
    if constexpr (NT) {
        asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen nt lds"
                     :
                     : "v"(voffset), "s"(rsrc), "s"(__builtin_amdgcn_readfirstlane(static_cast<int>(lds_base)))
                     : "memory", "m0");
    } else {
        asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                     :
                     : "v"(voffset), "s"(rsrc), "s"(__builtin_amdgcn_readfirstlane(static_cast<int>(lds_base)))
                     : "memory", "m0");
    }
}

// Same with 4 bytes per lane (LDS at `lds_base` + 4 * lane).
__device__ __forceinline__ void dma_lds4(const u32x4& rsrc, uint32_t lds_base, uint32_t voffset) {
    asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dword %0, %1, 0 offen lds"
                 :
                 : "v"(voffset), "s"(rsrc), "s"(__builtin_amdgcn_readfirstlane(static_cast<int>(lds_base)))
                 : "memory", "m0");
}

// Raw buffer descriptor over `bytes` bytes at `base` (stride 0, same flags as make_rsrc).
__device__ __forceinline__ u32x4 rsrc_words(const void* base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    const auto rfl = [](uint32_t x) {
        return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(x)));
    };
    return u32x4{rfl(static_cast<uint32_t>(a)), rfl(static_cast<uint32_t>(a >> 32) & 0xFFFFu), rfl(bytes),
                 0x00020000u};
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)(p)));
}

// Copies ROWS rows of a [rows, D] strided matrix (row stride `row_stride`
// elements) into a swizzled tile by direct HBM -> LDS loads; rows at or past
// `rows_valid` read as zero (buffer range check). The NW waves move 1 KB blocks
// of 8 (D = 64), 4 (D = 128) or 2 (D = 256) rows. NT: non-temporal copies (see
// dma_lds16).
template <int D, int NW, int ROWS, bool NT = false>
__device__ __forceinline__ void copy_rows_dma(const uint16_t* base, int64_t row_stride, int rows_valid,
                                              uint16_t* tile, int wave, int lane) {
    constexpr int CH = D / 8;
    constexpr int RPB = 64 / CH;
    constexpr int NBLK = ROWS / RPB;
    static_assert(NBLK % NW == 0, "tile blocks must divide among the waves");
    constexpr int IPW = NBLK / NW;
    const uint32_t row_bytes = static_cast<uint32_t>(row_stride) * 2u;
    const uint32_t bytes =
        rows_valid > 0 ? static_cast<uint32_t>((min(rows_valid, ROWS) - 1) * row_stride + D) * 2u : 0u;
    const u32x4 r = rsrc_words(base, bytes);
    const uint32_t tile_lds = lds_addr(tile);
    const int rr = lane / CH;
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
        const int blk = wave * IPW + i;
        const int gc = (lane % CH) ^ kv_swizzle<CH>(blk * RPB + rr);
        dma_lds16<NT>(r, tile_lds + blk * 1024u, static_cast<uint32_t>(blk * RPB + rr) * row_bytes + gc * 16u);
    }
}

// Per-lane parts of the swizzled tile addresses. The swizzle of a row depends
// only on row bits that the compile-time parts of the reads (32-row halves,
// 16-row groups) leave unchanged, so each read is the lane base plus a
// constant row offset plus 8 * (constant chunk ^ lane chunk key): one XOR.
template <int D>
struct TileLane {
    int rm_base;   // row-major read: row l32
    int rm_key;    // chunk key: hh ^ swizzle(l32)
    int tr_base;   // transposed read: row 4hh + li/4, 4-element half li & 1
    int tr_key_lo; // chunk key of that row: (2 g16 + (li & 3) / 2) ^ swizzle(row)
    int tr_key_hi; // same for the row 8 further down

    __device__ __forceinline__ TileLane(int lane) {
        constexpr int CH = D / 8;
        const int l32 = lane & 31, hh = lane >> 5, g16 = (lane >> 4) & 1, li = lane & 15;
        rm_base = l32 * D;
        rm_key = hh ^ kv_swizzle<CH>(l32);
        const int r0 = 4 * hh + (li >> 2);
        const int y = 2 * g16 + ((li & 3) >> 1);
        tr_base = r0 * D + 4 * (li & 1);
        tr_key_lo = y ^ kv_swizzle<CH>(r0);
        tr_key_hi = y ^ kv_swizzle<CH>(r0 + 8);
    }
    // Hides the keys from loop-invariant hoisting: each read then costs one XOR
    // instead of a register holding its precomputed address.
    __device__ __forceinline__ void refresh() {
        asm volatile("" : "+v"(rm_key), "+v"(tr_key_lo), "+v"(tr_key_hi));
    }
    // Row-major 16-byte read of row 32 * half + l32, chunk 2 * ks + hh.
    __device__ __forceinline__ u32x4 rm(const uint16_t* tile, int half, int ks) const {
        return *reinterpret_cast<const u32x4*>(tile + rm_base + 32 * half * D + 8 * ((2 * ks) ^ rm_key));
    }
    // A operand of X^T = M^T P: element (d, r) = tile[16 tt + r][32 db + d], read
    // transposed from rows 16tt + 4hh + li/4 and + 8.
    __device__ __forceinline__ u32x4 tr(const uint16_t* tile, int db, int tt) const {
        const uint16_t* p = tile + tr_base + 16 * tt * D;
        const uint2 lo = ds_read_tr16(p + 8 * ((4 * db) ^ tr_key_lo));
        const uint2 hi = ds_read_tr16(p + 8 * D + 8 * ((4 * db) ^ tr_key_hi));
        return u32x4{lo.x, lo.y, hi.x, hi.y};
    }
};

// The same reads with every per-lane part precomputed: one offset per K chunk
// pair and per V^T column block (D / 16 + D / 16 registers), so a read costs one
// add of the tile base, and the constant row offsets go into the instruction's
// offset field. Used where the registers are free (the ping-pong forward); each
// precomputed read saves the XOR and adds TileLane spends per read.
template <int D>
struct TileOffs {
    static constexpr int KS = D / 16;
    static constexpr int DB = D / 32;
    int k[KS];     // row-major read of row l32, chunk 2 ks + hh
    int vlo[DB];   // transposed read, rows 4 hh + li / 4, column block db
    int vhi[DB];   // same, 8 rows further down

    __device__ __forceinline__ TileOffs(int lane) {
        const TileLane<D> tl(lane);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) k[ks] = tl.rm_base + 8 * ((2 * ks) ^ tl.rm_key);
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            vlo[db] = tl.tr_base + 8 * ((4 * db) ^ tl.tr_key_lo);
            vhi[db] = tl.tr_base + 8 * D + 8 * ((4 * db) ^ tl.tr_key_hi);
        }
    }
    __device__ __forceinline__ u32x4 rm(const uint16_t* tile, int half, int ks) const {
        return *reinterpret_cast<const u32x4*>(tile + k[ks] + 32 * half * D);
    }
    __device__ __forceinline__ u32x4 tr(const uint16_t* tile, int db, int tt) const {
        const uint2 lo = ds_read_tr16(tile + vlo[db] + 16 * tt * D);
        const uint2 hi = ds_read_tr16(tile + vhi[db] + 16 * tt * D);
        return u32x4{lo.x, lo.y, hi.x, hi.y};
    }
};

constexpr int kBN = 64;               // keys per K/V tile of the forward kernels
constexpr float kRescaleSlack = 8.0f;  // log2 units the running max may lag behind

// Slot boundary: this wave's LDS reads are complete, then the block barrier.
// The asm memory clobber keeps memory operations on their side; the scheduling
// barriers keep every other instruction on its side too.
__device__ __forceinline__ void slot_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// s_waitcnt vmcnt(N) with expcnt / lgkmcnt at their maximum (gfx9 encoding:
// vmcnt bits 3:0 in bits 3:0, bits 5:4 in bits 15:14).
template <int N>
__device__ __forceinline__ void wait_vmem_le() {
    static_assert(N >= 0 && N < 64, "vmcnt immediate");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// ---------------------------------------------------------------------------
// Dropout: FlashAttention-2's Philox4x32-7 stream (flash-attn2-rs/src/device/
// dropout.rs:31-51). Element (query q, key k) of head bh = b * H + h is kept when
// byte ((q % 16) / 8 * 2 + k % 2) of word (k % 32) / 8 of
//     philox(seed, offset + 32 bh + 4 (q % 8) + (k % 8) / 2, row q / 16, col k / 32)
// is <= threshold (= floor(keep * 255)); rows and columns count from the start
// of the (varlen) sequence. The mapping is the reference's, fixed by its CUDA
// fragment layout; the kernels here evaluate it in their own layouts.
// ---------------------------------------------------------------------------
struct DropoutState {
    uint64_t seed;
    uint64_t offset;
    uint32_t threshold;
};

// Seed and offset from the device state tensor when given (read on the launch
// stream, so a captured graph replays the live values), else from the launch.
template <typename P>
__device__ __forceinline__ DropoutState dropout_state(const P& p) {
    DropoutState d;
    d.seed = p.rng_state ? static_cast<uint64_t>(p.rng_state[0]) : p.drop_seed;
    d.offset = p.rng_state ? static_cast<uint64_t>(p.rng_state[1]) : p.drop_offset;
    d.threshold = p.drop_threshold;
    return d;
}

__device__ __forceinline__ void philox4x32_7(uint64_t seed, uint64_t counter, uint32_t row, uint32_t col,
                                             uint32_t (&out)[4]) {
    uint32_t c0 = static_cast<uint32_t>(counter), c1 = static_cast<uint32_t>(counter >> 32);
    uint32_t c2 = row, c3 = col;
    uint32_t k0 = static_cast<uint32_t>(seed), k1 = static_cast<uint32_t>(seed >> 32);
#pragma unroll
    for (int i = 0; i < 7; ++i) {
        const uint64_t a = static_cast<uint64_t>(c0) * 0xD2511F53u;
        const uint64_t b = static_cast<uint64_t>(c2) * 0xCD9E8D57u;
        const uint32_t n0 = static_cast<uint32_t>(b >> 32) ^ c1 ^ k0;
        const uint32_t n2 = static_cast<uint32_t>(a >> 32) ^ c3 ^ k1;
        c1 = static_cast<uint32_t>(b);
        c3 = static_cast<uint32_t>(a);
        c0 = n0;
        c2 = n2;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0;
    out[1] = c1;
    out[2] = c2;
    out[3] = c3;
}

// Keep bits for a lane that owns query q and, of the 32-key block kblock, the
// 16 keys 8 (r / 4) + 4 hh + r % 4 (r = 0..15; the S^T accumulator layout of the
// forward and dQ kernels). Bit r set = kept.
__device__ __forceinline__ uint32_t keep_bits_query_lane(const DropoutState& d, uint32_t bh, uint32_t q,
                                                         uint32_t kblock, int hh) {
    const uint64_t base = d.offset + 32ull * bh + 4u * (q % 8u) + 2u * hh;
    uint32_t x0[4], x1[4];
    philox4x32_7(d.seed, base, q / 16u, kblock, x0);
    philox4x32_7(d.seed, base + 1, q / 16u, kblock, x1);
    const uint32_t rshift = ((q % 16u) / 8u) * 16u;
    uint32_t bits = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const uint32_t word = ((r & 3) >> 1) ? x1[r >> 2] : x0[r >> 2];
        const uint32_t byte = (word >> (rshift + 8u * (r & 1))) & 255u;
        bits |= (byte <= d.threshold ? 1u : 0u) << r;
    }
    return bits;
}

// Keep bits for a lane that owns key k and the 16 queries q0 + 8 (r / 4) + 4 hh +
// r % 4 of a 32-row chunk starting at q0 (a multiple of 16; the S = Q K^T
// accumulator layout of the dK/dV kernels). Bit r set = kept.
__device__ __forceinline__ uint32_t keep_bits_key_lane(const DropoutState& d, uint32_t bh, uint32_t q0,
                                                       uint32_t k, int hh) {
    const uint32_t word = (k % 32u) / 8u;
    const uint32_t kshift = 8u * (k & 1u);
    uint32_t bits = 0;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const uint32_t lane = 4u * (4u * hh + m) + (k % 8u) / 2u;
            uint32_t x[4];
            philox4x32_7(d.seed, d.offset + 32ull * bh + lane, q0 / 16u + rb, k / 32u, x);
            const uint32_t w = word == 0 ? x[0] : word == 1 ? x[1] : word == 2 ? x[2] : x[3];
            // r = 8 rb + m: query row % 16 = 4 hh + m (< 8); r = 8 rb + 4 + m: + 8.
            bits |= (((w >> kshift) & 255u) <= d.threshold ? 1u : 0u) << (8 * rb + m);
            bits |= (((w >> (16u + kshift)) & 255u) <= d.threshold ? 1u : 0u) << (8 * rb + 4 + m);
        }
    }
    return bits;
}

// keep_bits_query_lane for a wave whose lane l holds query q with q % 16 ==
// l % 16 (all 64 lanes active). The two Philox instances a lane needs (counter
// low bit t = 0, 1) are the same for lanes q and q ^ 8, which sit 8 apart in one
// 16-lane DPP row: each lane computes instance t = (q % 16) / 8 and takes the
// other from its partner with a row rotation by 8. Same bits as
// keep_bits_query_lane.
__device__ __forceinline__ uint32_t keep_bits_query_lane_shared(const DropoutState& d, uint32_t bh, uint32_t q,
                                                                uint32_t kblock, int hh) {
    const uint32_t own_t = (q % 16u) / 8u;
    uint32_t own[4], other[4];
    philox4x32_7(d.seed, d.offset + 32ull * bh + 4u * (q % 8u) + 2u * hh + own_t, q / 16u, kblock, own);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // DPP row_ror:8 (control 0x128): lane i of a 16-lane row reads lane (i + 8) % 16.
        other[i] = static_cast<uint32_t>(
            __builtin_amdgcn_update_dpp(0, static_cast<int>(own[i]), 0x128, 0xF, 0xF, false));
    }
    const uint32_t rshift = own_t * 16u;
    uint32_t bits = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const uint32_t t = static_cast<uint32_t>((r & 3) >> 1);
        const uint32_t word = t == own_t ? own[r >> 2] : other[r >> 2];
        const uint32_t byte = (word >> (rshift + 8u * (r & 1))) & 255u;
        bits |= (byte <= d.threshold ? 1u : 0u) << r;
    }
    return bits;
}

// Zeroes the dropped entries of the 16 scores a lane holds for query q of the
// 32-key block kblock (the S^T accumulator layout; element r is key
// 8 (r / 4) + 4 hh + r % 4): the keep decisions of keep_bits_query_lane_shared,
// applied directly. Of the two Philox words an element may come from, the lane
// computed one and lane l ^ 8 (same row of 16) the other; a DPP row_ror:8 move
// restricted to the banks (4-lane groups) that need the partner's word fetches
// it, so each element costs one byte extract, one compare and one select.
// Requires q % 16 == lane % 16.
__device__ __forceinline__ void apply_dropout_query_lane(const DropoutState& d, uint32_t bh, uint32_t q,
                                                         uint32_t kblock, int hh, f32x16& s) {
    const uint32_t own_t = (q % 16u) / 8u;
    uint32_t own[4];
    philox4x32_7(d.seed, d.offset + 32ull * bh + 4u * (q % 8u) + 2u * hh + own_t, q / 16u, kblock, own);
    const uint32_t rshift = own_t * 16u;
#pragma unroll
    for (int wi = 0; wi < 4; ++wi) {
        const int o = static_cast<int>(own[wi]);
        // Word of counter t = 0: lanes 8-15 of each row (banks 2, 3) take lane l - 8's.
        const uint32_t w0 = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(o, o, 0x128, 0xF, 0xC, false));
        // Word of counter t = 1: lanes 0-7 (banks 0, 1) take lane l + 8's.
        const uint32_t w1 = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(o, o, 0x128, 0xF, 0x3, false));
        const uint32_t h0 = w0 >> rshift, h1 = w1 >> rshift;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int r0 = 4 * wi + e, r1 = 4 * wi + 2 + e;
            s[r0] = ((h0 >> (8 * e)) & 255u) <= d.threshold ? s[r0] : 0.0f;
            s[r1] = ((h1 >> (8 * e)) & 255u) <= d.threshold ? s[r1] : 0.0f;
        }
    }
}

// keep_bits_key_lane for a wave whose lane l holds key k with k % 32 == l % 32
// (all 64 lanes active). The 8 Philox calls per lane above cover only 32
// distinct counters per half-wave: (m, rb) x (k % 8) / 2. Lane 8j + 2c + e of a
// half computes the instance (m = j, rb = e, c) once, and four exchange rounds
// of two ds_bpermute each deliver word (k % 32) / 8 of every instance a lane
// needs: in round s a lane publishes word (j + s) % 4 and reads the instances
// with m = (j - s) % 4. Same bits as keep_bits_key_lane.
__device__ __forceinline__ uint32_t keep_bits_key_lane_shared(const DropoutState& d, uint32_t bh, uint32_t q0,
                                                              uint32_t k, int hh) {
    const uint32_t l32 = k % 32u;
    const uint32_t j = l32 / 8u, c = (l32 % 8u) / 2u, e = l32 & 1u;
    uint32_t x[4];
    philox4x32_7(d.seed, d.offset + 32ull * bh + 4u * (4u * hh + j) + c, q0 / 16u + e, k / 32u, x);
    const uint32_t kshift = 8u * e;
    uint32_t bits = 0;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const uint32_t wi = (j + s) & 3u;
        const uint32_t pub = wi == 0 ? x[0] : wi == 1 ? x[1] : wi == 2 ? x[2] : x[3];
        const uint32_t m = (j - s) & 3u;
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
            const int src = 32 * hh + 8 * static_cast<int>(m) + 2 * static_cast<int>(c) + rb;
            const uint32_t w = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(4 * src, static_cast<int>(pub)));
            bits |= (((w >> kshift) & 255u) <= d.threshold ? 1u : 0u) << (8 * rb + m);
            bits |= (((w >> (16u + kshift)) & 255u) <= d.threshold ? 1u : 0u) << (8 * rb + 4 + m);
        }
    }
    return bits;
}

// ---------------------------------------------------------------------------
// Layout staging (layout.hip): what prepare_attention_tensor and the `out`
// copy of flash-attn2-rs/src/host/layout.rs:46-125 and host/forward/mod.rs:
// 349-376 do. An attention tensor whose rows the kernels cannot read as
// 16-byte vectors (base not 16-byte aligned, an outer stride not a multiple
// of 8 elements) or, for K/V, whose sequence rows overlap or are more than
// 2^23 elements apart, is copied into a packed buffer first; an output with
// such rows, or one overlapping an input, is written to a packed buffer and
// copied out afterwards. Buffers come from the stream-ordered allocator
// (hipMallocAsync / hipFreeAsync on the call's stream), as the reference takes
// them from its caller's allocator.
// ---------------------------------------------------------------------------
class Staged {
public:
    // `seq_dim` >= 0 adds the K/V sequence-row checks for that dimension
    // (head size `d`). With copy_in the tensor's values are copied into the
    // packed buffer (inputs); without, only the buffer is made (outputs).
    Staged(const kcr_tensor* t, hipStream_t s, bool copy_in, int seq_dim = -1, int64_t d = 0,
           std::initializer_list<const kcr_tensor*> must_not_overlap = {});
    ~Staged();
    Staged(const Staged&) = delete;
    Staged& operator=(const Staged&) = delete;
    const kcr_tensor* get() const { return buffer_ ? &packed_ : src_; }
    bool staged() const { return buffer_ != nullptr; }
    // Copies the packed buffer back into the caller's tensor (outputs).
    void copy_out();

private:
    const kcr_tensor* src_;
    kcr_tensor packed_{};
    void* buffer_ = nullptr;
    hipStream_t stream_;
};

// Diagnostic probabilities of a dropout forward (flash_probs.hip): fills the
// whole [batch, heads, rq, rk] plane `probs` (q's dtype, contiguous, rq and rk
// multiples of 128) from the inputs, masks, dropout state and the LSE the
// forward in `prm` wrote.
void launch_dropout_probabilities(const FwdParams& prm, bool varlen, int dtype, void* probs, int64_t rq,
                                  int64_t rk, hipStream_t s);

// A zero-padded, packed copy of an attention tensor whose last dimension is
// widened to `width` (inputs: copied in, the extra columns zero), or a padded
// output buffer whose first columns copy_out() writes back to the tensor.
// Head sizes the tiled kernels do not cover run on them through these copies.
class Padded {
public:
    Padded(const kcr_tensor* t, int64_t width, hipStream_t s, bool copy_in);
    ~Padded();
    Padded(const Padded&) = delete;
    Padded& operator=(const Padded&) = delete;
    const kcr_tensor* get() const { return src_ ? &padded_ : nullptr; }
    void copy_out();

private:
    const kcr_tensor* src_;
    kcr_tensor padded_{};
    void* buffer_ = nullptr;
    hipStream_t stream_;
};

// Whether two tensors' byte ranges intersect.
bool spans_overlap(const kcr_tensor* a, const kcr_tensor* b);

// Whether no two elements of `t` share an address (strides non-negative and,
// taken in increasing order, each at least the span of the dimensions below).
bool nonoverlapping_layout(const kcr_tensor* t);

}  // namespace attn
}  // namespace kcr
