// FlashAttention-2 forward on MI355X (gfx950): dense (`fwd`, `fwd_lse`) and packed
// variable-length (`varlen_fwd_explicit`) attention with GQA, causal / sliding
// windows, softcap and ALiBi.
//
// Reference semantics: flash-attn2-rs/src/device/forward/mod.rs:1162-1407 (core
// loop), :444-557 (scores and masks), :846-871 (LSE), device/config.rs:103-207
// (launch tile, GQA head mapping, key range), device/varlen/mod.rs:60-210 (per
// sequence bounds from cu_seqlens), host/forward/mod.rs:52-853 and
// host/varlen/mod.rs:21-670 (validation, window normalisation, empty inputs).
//
// MI355X design (shared by both kernels of this file)
//   * Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16
//     (bf16 or f16): the accumulator layout puts one query per lane (lane % 32)
//     and 16 keys per lane-half in registers, so the online-softmax row max is a
//     register reduction plus ONE cross-half exchange (lane ^ 32), and the row
//     sum needs no exchange until the end.
//   * The exponentiated scores are already laid out as the B operand of
//     O^T = V^T P^T: the accumulator registers are packed to bf16/f16 pairs in
//     place, no LDS round trip for P.
//   * Q stays in VGPRs for the whole key loop; keys stream in tiles of 64.
//   * Masks are evaluated only on tiles that cross a causal / window / sequence
//     edge; the online softmax rescales O lazily (only when a row max grows by
//     more than kRescaleSlack in log2 units).
//   * Causal grids run the longest query tiles first, and the query heads sharing
//     one KV head are placed on one XCD (blocks are dealt round-robin over the 8
//     XCDs) so their K/V tiles hit the same L2.
//
// flash_fwd_tiled_kernel (head sizes 64, 128 and 256, plain or with softcap /
// ALiBi) copies K/V tiles HBM -> LDS with direct buffer loads into swizzled
// row-major tiles; flash_fwd_kernel (other head sizes, non-positive scales)
// stages the tiles through registers and stores V transposed.

#include "attention.h"

#include <algorithm>
#include <mutex>
#include <type_traits>
#include <vector>

namespace kcr {
namespace attn {


// V^T tile rows hold 16 chunks of 4 keys (8 bytes). The loading threads write
// one chunk to each of 16 rows that are 8 apart; XOR-ing the chunk index with
// bits of (row / 16) spreads those writes over distinct LDS banks. Bit 1 of
// the chunk index is left alone so the two chunks an MFMA operand needs
// (chunks c and c + 2) stay a constant 16 bytes apart.
__device__ __forceinline__ int vt_swizzle(int row) {
    const int x = (row >> 4) & 7;
    return (x & 1) | ((x & 6) << 1);
}
constexpr int kLookTiled = 3;          // operand reads in flight ahead of their MFMA (tiled kernel)

// GENERAL covers softcap, ALiBi and head sizes below the compiled bucket (zeroed
// lanes of the padded head dimension); the fast path is the plain scaled dot
// product with a positive scale.
template <typename T, int D, int QT, int NW, bool VARLEN, bool GENERAL>
__global__ void __launch_bounds__(NW * 64, QT == 1 ? 2 : 1) flash_fwd_kernel(const FwdParams p) {
    constexpr int BN = kBN;
    constexpr int BM = 32 * QT * NW;
    constexpr int NT = NW * 64;
    constexpr int KS = D / 16;   // MFMA k-steps over the head dim
    constexpr int DB = D / 32;   // 32-wide blocks of the head dim in O
    constexpr int KSTR = D + 8;  // K tile row stride in LDS (elements)
    constexpr int VSTR = BN + 8; // V^T tile row stride in LDS (elements)
    constexpr int DCH = D / 8;   // 16-byte chunks per row
    constexpr int KCH = BN * DCH;
    constexpr int KPT = (KCH + NT - 1) / NT;
    constexpr int VIT = (BN / 4) * DCH;
    constexpr int VPT = (VIT + NT - 1) / NT;
    constexpr int KTILE = BN * KSTR;
    constexpr int VTILE = D * VSTR;

    // Two stages of (K, V^T) so one barrier per key tile suffices.
    __shared__ __attribute__((aligned(16))) uint16_t k_lds[2 * KTILE];
    __shared__ __attribute__((aligned(16))) uint16_t v_lds[2 * VTILE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int l32 = lane & 31;
    const int hh = lane >> 5;

    // ---- block -> (batch, head, query tile) ----
    const int per_tile = p.batch * p.heads;
    const int qo = blockIdx.x / per_tile;
    const int rem = blockIdx.x - qo * per_tile;
    int bh;
    if (p.xcd_groups) {
        const int xcd = rem & 7;
        const int rr = rem >> 3;
        const int j = rr % p.gqa;
        const int g = (rr / p.gqa) * 8 + xcd;
        bh = g * p.gqa + j;
    } else {
        bh = rem;
    }
    const int b = bh / p.heads;
    const int head = bh - b * p.heads;
    const int kvh = head / p.gqa;
    const DropoutState drop = p.drop_threshold < 255 ? dropout_state(p) : DropoutState{};
    // Longest causal tiles first: block qo takes the qo-th query tile counted
    // from the end of its own sequence (varlen sequences end at different tiles).
    int qb = p.q_blocks - 1 - qo;

    int64_t q_off = 0, k_off = 0;
    int sq = p.seqlen_q, sk = p.seqlen_k;
    int lse_row0 = 0;
    [[maybe_unused]] int part_row0 = 0;  // row of the split partials (packed row index)
    int64_t k_batch = 0;
    if constexpr (VARLEN) {
        const VarSeq vs = varlen_seq(p, b);
        if (!vs.ok) return;
        sq = vs.sq;
        sk = vs.sk;
        q_off = p.rows_per_seq ? 0 : static_cast<int64_t>(vs.qs);
        k_off = vs.k_row0;
        k_batch = vs.k_batch;
        lse_row0 = static_cast<int>(q_off);
        part_row0 = vs.qs;
        qb = (sq + BM - 1) / BM - 1 - qo;
        if (qb < 0) return;
    }
    const int row0 = qb * BM;
    if (row0 >= sq) return;
    const int off = sk - sq;
    const int wl = p.window_left;
    const int wr = p.window_right;

    const uint16_t* qbase;
    const uint16_t* kbase;
    const uint16_t* vbase;
    uint16_t* obase;
    if constexpr (VARLEN) {
        qbase = static_cast<const uint16_t*>(p.q) + b * p.q_b + q_off * p.q_s + head * p.q_h;
        kbase = static_cast<const uint16_t*>(p.k) + k_batch * p.k_b + k_off * p.k_s + kvh * p.k_h;
        vbase = static_cast<const uint16_t*>(p.v) + k_batch * p.v_b + k_off * p.v_s + kvh * p.v_h;
        obase = static_cast<uint16_t*>(p.o) + b * p.o_b + q_off * p.o_s + head * p.o_h;
    } else {
        qbase = static_cast<const uint16_t*>(p.q) + b * p.q_b + head * p.q_h;
        kbase = static_cast<const uint16_t*>(p.k) + b * p.k_b + kvh * p.k_h;
        vbase = static_cast<const uint16_t*>(p.v) + b * p.v_b + kvh * p.v_h;
        obase = static_cast<uint16_t*>(p.o) + b * p.o_b + head * p.o_h;
    }
    float* lse_base = p.lse + b * p.lse_b + head * p.lse_h + lse_row0;

    // ---- key range of this query tile (device/config.rs:183-207) ----
    const int last_row = min(row0 + BM, sq) - 1;
    int kv_end = sk;
    if (wr >= 0) kv_end = max(0, min(sk, last_row + 1 + off + wr));
    int kv_begin = 0;
    if (wl >= 0) kv_begin = (max(0, min(sk, row0 + off - wl)) / BN) * BN;

    // ---- Q fragments in registers: B operand of S^T = K Q^T ----
    const int wrow0 = row0 + wave * 32 * QT;
    u32x4 qf[QT][KS];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int row = wrow0 + qt * 32 + l32;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int d0 = 16 * ks + 8 * hh;
            if (row < sq && (!GENERAL || d0 < p.head_dim)) {
                qf[qt][ks] = *reinterpret_cast<const u32x4*>(qbase + row * p.q_s + d0);
            } else {
                qf[qt][ks] = u32x4{0, 0, 0, 0};
            }
        }
    }

    float slope_log2 = 0.0f;
    if constexpr (GENERAL) {
        if (p.alibi) slope_log2 = p.alibi[b * p.alibi_b + head] * kLog2e;
    }
    // Fast path: exp2(s * c - m) with the scale folded into one FMA.
    const float c = GENERAL ? 1.0f : p.scale_log2;

    f32x16 o[QT][DB];
    float m[QT], l[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        m[qt] = -INFINITY;
        l[qt] = 0.0f;
#pragma unroll
        for (int db = 0; db < DB; ++db) o[qt][db] = f32x16{};
    }

    // ---- tile staging: HBM -> registers (buffer loads, rows past the end read
    // as zero) -> LDS ----
    u32x4 kreg[KPT];
    u32x4 vreg[VPT][4];
    const uint32_t krow_bytes = static_cast<uint32_t>(p.k_s) * 2u;
    const uint32_t vrow_bytes = static_cast<uint32_t>(p.v_s) * 2u;
    auto load_tile = [&](int kb) {
        // Valid bytes from the tile's first row: rows >= sk (and the padded head
        // dims of the last row) fall outside the range and read as zero.
        int rows = min(sk - kb, BN);
        const uint16_t* kt = kbase + static_cast<int64_t>(kb) * p.k_s;
        const uint16_t* vt = vbase + static_cast<int64_t>(kb) * p.v_s;
        if constexpr (VARLEN) {
            if (p.block_table) {
                const int64_t page = page_of(p, b, kb);
                const int64_t within = kb % p.page_size;
                kt = kbase + page * p.k_page + within * p.k_s;
                vt = vbase + page * p.v_page + within * p.v_s;
                if (page < 0) rows = 0;
            }
        }
        const uint32_t kbytes = rows > 0 ? static_cast<uint32_t>((rows - 1) * p.k_s + p.head_dim) * 2u : 0u;
        const uint32_t vbytes = rows > 0 ? static_cast<uint32_t>((rows - 1) * p.v_s + p.head_dim) * 2u : 0u;
        const auto kr = make_rsrc(kt, kbytes);
        const auto vr = make_rsrc(vt, vbytes);
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int cidx = tid + i * NT;
            if (KCH % NT == 0 || cidx < KCH) {
                const int key = cidx / DCH;
                const int dc = cidx - key * DCH;
                kreg[i] = buffer_load16(kr, key * krow_bytes + dc * 16);
                if constexpr (GENERAL) {
                    if (dc * 8 >= p.head_dim) kreg[i] = u32x4{0, 0, 0, 0};
                }
            }
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int it = tid + i * NT;
            if (VIT % NT == 0 || it < VIT) {
                const int kq = it / DCH;
                const int dc = it - kq * DCH;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    vreg[i][e] = buffer_load16(vr, (4 * kq + e) * vrow_bytes + dc * 16);
                    if constexpr (GENERAL) {
                        if (dc * 8 >= p.head_dim) vreg[i][e] = u32x4{0, 0, 0, 0};
                    }
                }
            }
        }
    };
    auto store_tile = [&](int stage) {
        uint16_t* kl = k_lds + stage * KTILE;
        uint16_t* vl = v_lds + stage * VTILE;
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int cidx = tid + i * NT;
            if (KCH % NT == 0 || cidx < KCH) {
                const int key = cidx / DCH;
                const int dc = cidx - key * DCH;
                *reinterpret_cast<u32x4*>(&kl[key * KSTR + dc * 8]) = kreg[i];
            }
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int it = tid + i * NT;
            if (VIT % NT == 0 || it < VIT) {
                const int kq = it / DCH;
                const int dc = it - kq * DCH;
                // 4 keys x 8 d -> eight 8-byte rows of V^T (byte permutes).
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const uint32_t a0 = vreg[i][0][w], a1 = vreg[i][1][w];
                    const uint32_t a2 = vreg[i][2][w], a3 = vreg[i][3][w];
                    uint2 lo, hi;  // d = 2w (low halves) and d = 2w + 1 (high halves)
                    lo.x = __builtin_amdgcn_perm(a1, a0, 0x05040100u);
                    lo.y = __builtin_amdgcn_perm(a3, a2, 0x05040100u);
                    hi.x = __builtin_amdgcn_perm(a1, a0, 0x07060302u);
                    hi.y = __builtin_amdgcn_perm(a3, a2, 0x07060302u);
                    const int r0 = 8 * dc + 2 * w;
                    *reinterpret_cast<uint2*>(&vl[r0 * VSTR + 4 * (kq ^ vt_swizzle(r0))]) = lo;
                    *reinterpret_cast<uint2*>(&vl[(r0 + 1) * VSTR + 4 * (kq ^ vt_swizzle(r0 + 1))]) = hi;
                }
            }
        }
    };

    const int ntiles = kv_begin < kv_end ? (kv_end - kv_begin + BN - 1) / BN : 0;
    if (ntiles > 0) {
        load_tile(kv_begin);
        store_tile(0);
        if (ntiles > 1) load_tile(kv_begin + BN);
        __syncthreads();
    }

    for (int t = 0; t < ntiles; ++t) {
        const int kb = kv_begin + t * BN;
        const uint16_t* kl = k_lds + (t & 1) * KTILE;
        const uint16_t* vl = v_lds + (t & 1) * VTILE;

        // ---- S^T = K Q^T for 64 keys x 32*QT queries ----
        f32x16 s[QT][2];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            s[qt][0] = f32x16{};
            s[qt][1] = f32x16{};
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const u32x4 ka0 = *reinterpret_cast<const u32x4*>(&kl[l32 * KSTR + 16 * ks + 8 * hh]);
            const u32x4 ka1 = *reinterpret_cast<const u32x4*>(&kl[(32 + l32) * KSTR + 16 * ks + 8 * hh]);
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                s[qt][0] = mfma32<T>(ka0, qf[qt][ks], s[qt][0]);
                s[qt][1] = mfma32<T>(ka1, qf[qt][ks], s[qt][1]);
            }
        }

        // The next tile's registers go to the other LDS stage while this one is
        // consumed; its last readers finished before the previous barrier.
        if (t + 1 < ntiles) {
            store_tile((t + 1) & 1);
            if (t + 2 < ntiles) load_tile(kb + 2 * BN);
        }

        // ---- scores, masks, online softmax (lazy rescale) ----
        const bool need_mask = (kb + BN > sk) || (wr >= 0 && kb + BN - 1 > row0 + off + wr) ||
                               (wl >= 0 && kb < last_row + off - wl);
        u32x4 pk[QT][4];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            const int row = wrow0 + qt * 32 + l32;
            if constexpr (GENERAL) {
#pragma unroll
                for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int col = kb + 32 * sub + 8 * (r >> 2) + 4 * hh + (r & 3);
                        float x = s[qt][sub][r];
                        if (p.tanh_scale > 0.0f) {
                            x = tanhf(x * p.tanh_scale) * p.scale_eff_log2;
                        } else {
                            x *= p.scale_log2;
                        }
                        if (p.alibi) {
                            x += p.alibi_causal ? slope_log2 * static_cast<float>(col)
                                                : -slope_log2 * fabsf(static_cast<float>(row + off - col));
                        }
                        s[qt][sub][r] = x;
                    }
                }
            }
            if (need_mask) {
#pragma unroll
                for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int col = kb + 32 * sub + 8 * (r >> 2) + 4 * hh + (r & 3);
                        const bool masked = (col >= sk) || (wr >= 0 && col > row + off + wr) ||
                                            (wl >= 0 && col < row + off - wl);
                        s[qt][sub][r] = masked ? -INFINITY : s[qt][sub][r];
                    }
                }
            }
            float mx = lane_max32(s[qt][0], s[qt][1]);
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float m2 = mx * c;
            // Rescale O and l only when some row's max grew by more than the slack:
            // exp2(s*c - m) then stays <= 2^slack, which bf16 P and f32 sums hold.
            if (__any(m2 > m[qt] + kRescaleSlack)) {
                const float m_new = fmaxf(m[qt], m2);
                const float alpha = (m_new == -INFINITY) ? 1.0f : fast_exp2(m[qt] - m_new);
                m[qt] = m_new;
                l[qt] *= alpha;
#pragma unroll
                for (int db = 0; db < DB; ++db) o[qt][db] *= alpha;
            }
            const float neg_m = (m[qt] == -INFINITY) ? 0.0f : -m[qt];
            float rowsum = 0.0f;
#pragma unroll
            for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float pv = fast_exp2(__builtin_fmaf(s[qt][sub][r], c, neg_m));
                    s[qt][sub][r] = pv;
                    rowsum += pv;
                }
            }
            l[qt] += rowsum;
            if (p.drop_threshold < 255) {
                // Dropout after the (undropped) row sum: P and O only.
#pragma unroll
                for (int sub = 0; sub < 2; ++sub) {
                    const uint32_t bits = keep_bits_query_lane(drop, static_cast<uint32_t>(bh),
                                                               static_cast<uint32_t>(row),
                                                               static_cast<uint32_t>(kb / 32 + sub), hh);
#pragma unroll
                    for (int r = 0; r < 16; ++r) s[qt][sub][r] = ((bits >> r) & 1u) ? s[qt][sub][r] : 0.0f;
                }
            }
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) {
                const int sub = tt >> 1;
                const int base = 8 * (tt & 1);
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    pk[qt][tt][w] = pack2<T>(s[qt][sub][base + 2 * w], s[qt][sub][base + 2 * w + 1]);
                }
            }
        }

        // ---- O^T += V^T P^T ----
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) {
                const int vr = 32 * db + l32;
                const uint16_t* vrow = &vl[vr * VSTR + 4 * ((4 * tt + hh) ^ vt_swizzle(vr))];
                const uint2 lo = *reinterpret_cast<const uint2*>(vrow);
                const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 8);
                const u32x4 va = u32x4{lo.x, lo.y, hi.x, hi.y};
#pragma unroll
                for (int qt = 0; qt < QT; ++qt) o[qt][db] = mfma32<T>(va, pk[qt][tt], o[qt][db]);
            }
        }
        __syncthreads();
    }

    // ---- epilogue: O / l, LSE = (m + log2 l) * ln 2 (forward/mod.rs:846-865) ----
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int row = wrow0 + qt * 32 + l32;
        const float lt = l[qt] + __shfl_xor(l[qt], 32, 64);
        if (row >= sq) continue;
        const float inv = (lt > 0.0f ? 1.0f / lt : 0.0f) * (p.drop_threshold < 255 ? p.inv_keep : 1.0f);
        uint16_t* orow = obase + row * p.o_s;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = 32 * db + 8 * g + 4 * hh;
                if (!GENERAL || d < p.head_dim) {
                    uint2 w;
                    w.x = pack2<T>(o[qt][db][4 * g] * inv, o[qt][db][4 * g + 1] * inv);
                    w.y = pack2<T>(o[qt][db][4 * g + 2] * inv, o[qt][db][4 * g + 3] * inv);
                    *reinterpret_cast<uint2*>(orow + d) = w;
                }
            }
        }
        if (hh == 0) lse_base[row] = lt > 0.0f ? (m[qt] + fast_log2(lt)) * kLn2 : INFINITY;
    }
}

// ---------------------------------------------------------------------------
// Tiled forward (head size 64, 128 or 256). One block =
// 4 waves = 128 query rows of one head; each wave owns 32 rows, their Q in
// registers as the B operand of S^T = K Q^T (one query per lane: the row max and
// sum are in-lane reductions plus one cross-half shuffle). K and V tiles of 64
// keys (32 at D = 256) are copied HBM -> LDS by direct buffer loads into row-major tiles with
// XOR-swizzled 16-byte chunks (no staging registers, no VALU); K is read with
// ds_read_b128 and V^T, the A operand of O^T = V^T P^T, with ds_read_b64_tr_b16
// from the same row-major tile. Two blocks per CU at every head size. P^T stays
// in registers: the fp32 scores are
// packed in place into the B operand of the PV MFMA. Two LDS stages, the next
// tile's copy in flight during the current tile, one barrier per tile. STREAM:
// every K/V tile is read by this block only (cache decode with grouped rows),
// so the copies are non-temporal. SCORED: the scores are transformed before
// the softmax (softcap tanh and / or the ALiBi bias, in log2 units), which
// then runs with the scale already applied.
// ---------------------------------------------------------------------------
template <typename T, int D, bool VARLEN, bool DROPOUT, bool STREAM, bool SCORED = false>
__global__ void __launch_bounds__(256, 2) flash_fwd_tiled_kernel(const FwdParams p) {
    constexpr int NW = 4;
    // D = 256 takes 32-key tiles: O (128), Q (64) and S (16) registers then fit
    // two waves per SIMD, and 64 KB of tiles two blocks per CU.
    constexpr int BN = D > 128 ? 32 : kBN;
    constexpr int NSUB = BN / 32;  // 32-key halves of a tile
    constexpr int BM = 32 * NW;
    constexpr int KS = D / 16;
    constexpr int DB = D / 32;
    constexpr int TILE = BN * D;

    __shared__ __attribute__((aligned(1024))) uint16_t k_lds[2 * TILE];
    __shared__ __attribute__((aligned(1024))) uint16_t v_lds[2 * TILE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar copy addresses
    const int l32 = lane & 31;
    const int hh = lane >> 5;
    TileLane<D> tl(lane);

    // Query-tile-major grid, longest causal tiles first; with xcd_groups the
    // query heads of one KV head share blockIdx % 8, i.e. one XCD and its L2.
    // Split-KV grids (packed sequences only): the splits of one query tile are
    // adjacent blocks.
    const int nsplit = p.n_splits > 1 ? p.n_splits : 1;
    const int bid = static_cast<int>(blockIdx.x) / nsplit;
    const int split = static_cast<int>(blockIdx.x) - bid * nsplit;
    int b, head, qo;
    if (p.seq_major) {
        // Sequence-major (unmasked or packed grids): the blocks of one sequence
        // run together and share its K/V tiles in L2; the query heads of one KV
        // head keep one XCD when Hk is a multiple of 8.
        const int per_seq = p.q_blocks * p.heads;
        b = bid / per_seq;
        const int rem = bid - b * per_seq;
        qo = rem / p.heads;
        const int idx = rem - qo * p.heads;
        head = (idx % p.kv_heads) * p.gqa + idx / p.kv_heads;
    } else if (p.xcd_groups) {
        // Group-major per XCD (blocks go to XCD blockIdx % 8): each XCD runs
        // the query tiles of one (batch, KV head) group, longest first over its
        // query heads, before the next group, so one group's K/V tiles are live
        // in the XCD's L2 at a time.
        const int xcd = bid & 7;
        const int k = bid >> 3;
        const int per_group = p.q_blocks * p.gqa;
        const int gl = k / per_group;
        const int t = k - gl * per_group;
        qo = t / p.gqa;
        const int j = t - qo * p.gqa;
        const int bh = (gl * 8 + xcd) * p.gqa + j;
        b = bh / p.heads;
        head = bh - b * p.heads;
    } else {
        const int per_tile = p.batch * p.heads;
        qo = bid / per_tile;
        const int bh = bid - qo * per_tile;
        b = bh / p.heads;
        head = bh - b * p.heads;
    }
    const int kvh = head / p.gqa;
    const uint32_t bh = static_cast<uint32_t>(b * p.heads + head);
    DropoutState drop{};
    if constexpr (DROPOUT) drop = dropout_state(p);
    // Block qo takes the qo-th query tile counted from the end of its sequence
    // (varlen sequences end at different tiles).
    int qb = p.q_blocks - 1 - qo;

    int64_t q_off = 0, k_off = 0;
    int sq = p.seqlen_q, sk = p.seqlen_k;
    int lse_row0 = 0;
    int part_row0 = 0;  // row of the split partials (packed row index)
    int64_t k_batch = 0;
    if constexpr (VARLEN) {
        const VarSeq vs = varlen_seq(p, b);
        if (!vs.ok) {
            // Batched split partials have no fill: mark this block's rows as
            // unseen (LSE -inf) so the merge gives O = 0, LSE = +inf.
            if (nsplit > 1 && p.rows_per_seq > 0) {
                const int r = (p.q_blocks - 1 - qo) * BM + wave * 32 + l32;
                if (hh == 0 && r < p.rows_per_seq) {
                    p.lse_part[(static_cast<int64_t>(split) * p.heads + head) * p.total_q +
                               static_cast<int64_t>(b) * p.rows_per_seq + r] = -INFINITY;
                }
            }
            return;
        }
        sq = vs.sq;
        sk = vs.sk;
        q_off = p.rows_per_seq ? 0 : static_cast<int64_t>(vs.qs);
        k_off = vs.k_row0;
        k_batch = vs.k_batch;
        lse_row0 = static_cast<int>(q_off);
        part_row0 = vs.qs;
        qb = (sq + BM - 1) / BM - 1 - qo;
        if (qb < 0) return;
    } else {
        part_row0 = b * sq;  // dense split partials: packed row b * Sq + row
    }
    const int row0 = qb * BM;
    if (row0 >= sq) return;
    const int off = sk - sq;
    const int wl = p.window_left;
    const int wr = p.window_right;

    const uint16_t* qbase;
    const uint16_t* kbase;
    const uint16_t* vbase;
    uint16_t* obase;
    if constexpr (VARLEN) {
        qbase = static_cast<const uint16_t*>(p.q) + b * p.q_b + q_off * p.q_s + head * p.q_h;
        kbase = static_cast<const uint16_t*>(p.k) + k_batch * p.k_b + k_off * p.k_s + kvh * p.k_h;
        vbase = static_cast<const uint16_t*>(p.v) + k_batch * p.v_b + k_off * p.v_s + kvh * p.v_h;
        obase = static_cast<uint16_t*>(p.o) + b * p.o_b + q_off * p.o_s + head * p.o_h;
    } else {
        qbase = static_cast<const uint16_t*>(p.q) + b * p.q_b + head * p.q_h;
        kbase = static_cast<const uint16_t*>(p.k) + b * p.k_b + kvh * p.k_h;
        vbase = static_cast<const uint16_t*>(p.v) + b * p.v_b + kvh * p.v_h;
        obase = static_cast<uint16_t*>(p.o) + b * p.o_b + head * p.o_h;
    }
    float* lse_base = p.lse + b * p.lse_b + head * p.lse_h + lse_row0;

    const int last_row = min(row0 + BM, sq) - 1;
    int kv_end = sk;
    if (wr >= 0) kv_end = max(0, min(sk, last_row + 1 + off + wr));
    int kv_begin = 0;
    if (wl >= 0) kv_begin = (max(0, min(sk, row0 + off - wl)) / BN) * BN;

    const int row = row0 + wave * 32 + l32;
    u32x4 qf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        qf[ks] = row < sq ? *reinterpret_cast<const u32x4*>(qbase + row * p.q_s + 16 * ks + 8 * hh)
                          : u32x4{0, 0, 0, 0};
    }
    // Fast path: exp2(s * c - m) with the scale folded into one FMA; scored
    // tiles carry the scale (and bias) in the scores themselves.
    const float c = SCORED ? 1.0f : p.scale_log2;
    [[maybe_unused]] float slope_log2 = 0.0f;
    if constexpr (SCORED) {
        if (p.alibi) slope_log2 = p.alibi[b * p.alibi_b + head] * kLog2e;
    }

    f32x16 o[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db] = f32x16{};
    float m = -INFINITY, l = 0.0f;

    auto copy_tile = [&](int kb, int stage) {
        const uint16_t* kt = kbase + static_cast<int64_t>(kb) * p.k_s;
        const uint16_t* vt = vbase + static_cast<int64_t>(kb) * p.v_s;
        int rows = sk - kb;
        if constexpr (VARLEN) {
            if (p.block_table) {
                const int64_t page = page_of(p, b, kb);
                const int64_t within = kb % p.page_size;
                kt = kbase + page * p.k_page + within * p.k_s;
                vt = vbase + page * p.v_page + within * p.v_s;
                if (page < 0) rows = 0;
            }
        }
        copy_rows_dma<D, NW, BN, STREAM>(kt, p.k_s, rows, k_lds + stage * TILE, wave, lane);
        copy_rows_dma<D, NW, BN, STREAM>(vt, p.v_s, rows, v_lds + stage * TILE, wave, lane);
    };

    int ntiles = kv_begin < kv_end ? (kv_end - kv_begin + BN - 1) / BN : 0;
    if (nsplit > 1) {
        // This split's share of the key tiles (possibly none).
        const int per = (ntiles + nsplit - 1) / nsplit;
        const int lo = min(ntiles, split * per);
        kv_begin += lo * BN;
        ntiles = min(ntiles, lo + per) - lo;
    }
    if (ntiles > 0) {
        copy_tile(kv_begin, 0);
        wait_vmem();
        __syncthreads();
    }

    for (int t = 0; t < ntiles; ++t) {
        const int kb = kv_begin + t * BN;
        const uint16_t* kl = k_lds + (t & 1) * TILE;
        const uint16_t* vl = v_lds + (t & 1) * TILE;
        if (t + 1 < ntiles) copy_tile(kb + BN, (t + 1) & 1);
        if constexpr (STREAM) {
            // Waves whose rows all lie past the sequence (3 of 4 with 4 grouped
            // decode rows) only share the copies and the barrier.
            if (row0 + wave * 32 >= sq) {
                wait_vmem();
                __syncthreads();
                continue;
            }
        }

        // S^T = K Q^T for the 64 keys of the tile (two 32-key halves); the K
        // reads run kLookTiled MFMAs ahead of their use.
        f32x16 s[NSUB];
#pragma unroll
        for (int sub = 0; sub < NSUB; ++sub) s[sub] = f32x16{};
        {
            constexpr int N = NSUB * KS;
            u32x4 ring[kLookTiled];
            static_for<0, kLookTiled>([&](auto ic) __attribute__((always_inline)) {
                constexpr int i = decltype(ic)::value;
                ring[i] = tl.rm(kl, i % NSUB, i / NSUB);
            });
            __builtin_amdgcn_sched_group_barrier(0x100, kLookTiled, 0);
            static_for<0, N>([&](auto ic) __attribute__((always_inline)) {
                constexpr int i = decltype(ic)::value;
                const u32x4 a = ring[i % kLookTiled];
                if constexpr (i + kLookTiled < N) {
                    ring[i % kLookTiled] = tl.rm(kl, (i + kLookTiled) % NSUB, (i + kLookTiled) / NSUB);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                s[i % NSUB] = mfma32<T>(a, qf[i / NSUB], s[i % NSUB]);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            });
        }

        if constexpr (SCORED) {
            // The general kernel's score transform, with tanh from tanh_exp2.
            const bool cap = p.tanh_scale > 0.0f;
#pragma unroll
            for (int sub = 0; sub < NSUB; ++sub) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int col = kb + 32 * sub + 8 * (r >> 2) + 4 * hh + (r & 3);
                    float x = s[sub][r];
                    x = cap ? tanh_exp2(x * p.tanh_scale) * p.scale_eff_log2 : x * p.scale_log2;
                    if (p.alibi) {
                        x += p.alibi_causal ? slope_log2 * static_cast<float>(col)
                                            : -slope_log2 * fabsf(static_cast<float>(row + off - col));
                    }
                    s[sub][r] = x;
                }
            }
        }
        const bool need_mask = (kb + BN > sk) || (wr >= 0 && kb + BN - 1 > row0 + off + wr) ||
                               (wl >= 0 && kb < last_row + off - wl);
        if (need_mask) {
#pragma unroll
            for (int sub = 0; sub < NSUB; ++sub) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int col = kb + 32 * sub + 8 * (r >> 2) + 4 * hh + (r & 3);
                    const bool masked = (col >= sk) | (wr >= 0 & col > row + off + wr) |
                                        (wl >= 0 & col < row + off - wl);
                    s[sub][r] = masked ? -INFINITY : s[sub][r];
                }
            }
        }
        float mx = lane_max32(s[0], s[NSUB - 1]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m2 = mx * c;
        // Lazy rescale: the running max moves only when some row's max grows by
        // more than the slack (wave-uniform decision).
        if (__any(m2 > m + kRescaleSlack)) {
            const float m_new = fmaxf(m, m2);
            const float alpha = (m_new == -INFINITY) ? 1.0f : fast_exp2(m - m_new);
            m = m_new;
            l *= alpha;
#pragma unroll
            for (int db = 0; db < DB; ++db) o[db] *= alpha;
        }
        const float neg_m = (m == -INFINITY) ? 0.0f : -m;
        float rowsum = 0.0f;
#pragma unroll
        for (int sub = 0; sub < NSUB; ++sub) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float pv = fast_exp2(__builtin_fmaf(s[sub][r], c, neg_m));
                s[sub][r] = pv;
                rowsum += pv;
            }
        }
        l += rowsum;
        if constexpr (DROPOUT) {
            // The row sum above is of the undropped probabilities; dropped ones
            // leave P (and O) only.
#pragma unroll
            for (int sub = 0; sub < NSUB; ++sub) {
                apply_dropout_query_lane(drop, bh, static_cast<uint32_t>(row), static_cast<uint32_t>(kb / 32 + sub),
                                         hh, s[sub]);
            }
        }
        // P^T packed in place: k-slot j of group tt is key 16tt + 8(j/4) + 4hh + j%4.
        u32x4 pk[2 * NSUB];
#pragma unroll
        for (int tt = 0; tt < 2 * NSUB; ++tt) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                pk[tt][w] = pack2<T>(s[tt >> 1][8 * (tt & 1) + 2 * w], s[tt >> 1][8 * (tt & 1) + 2 * w + 1]);
            }
        }
        // O^T += V^T P^T (step i: db = i % DB, tt = i / DB), reads ahead as above.
        {
            constexpr int N = 2 * NSUB * DB;
            u32x4 ring[kLookTiled];
            static_for<0, kLookTiled>([&](auto ic) __attribute__((always_inline)) {
                constexpr int i = decltype(ic)::value;
                ring[i] = tl.tr(vl, i % DB, i / DB);
            });
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * kLookTiled, 0);
            static_for<0, N>([&](auto ic) __attribute__((always_inline)) {
                constexpr int i = decltype(ic)::value;
                const u32x4 a = ring[i % kLookTiled];
                if constexpr (i + kLookTiled < N) {
                    ring[i % kLookTiled] = tl.tr(vl, (i + kLookTiled) % DB, (i + kLookTiled) / DB);
                    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                }
                o[i % DB] = mfma32<T>(a, pk[i / DB], o[i % DB]);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            });
        }
        wait_vmem();
        __syncthreads();
    }

    const float lt = l + __shfl_xor(l, 32, 64);
    if (nsplit > 1) {
        // fp32 partials of this split: O normalised by its own row sum, LSE
        // -inf when the split saw no key of the row.
        if (row < sq) {
            const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
            const int64_t prow = (static_cast<int64_t>(split) * p.heads + head) * p.total_q + part_row0 + row;
            float* op = p.o_part + prow * D;
#pragma unroll
            for (int db = 0; db < DB; ++db) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int d = 32 * db + 8 * g + 4 * hh;
                    *reinterpret_cast<float4*>(op + d) = float4{o[db][4 * g] * inv, o[db][4 * g + 1] * inv,
                                                                o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv};
                }
            }
            if (hh == 0) p.lse_part[prow] = lt > 0.0f ? (m + fast_log2(lt)) * kLn2 : -INFINITY;
        }
        return;
    }
    if (row < sq) {
        const float inv = (lt > 0.0f ? 1.0f / lt : 0.0f) * (DROPOUT ? p.inv_keep : 1.0f);
        uint16_t* orow = obase + row * p.o_s;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = 32 * db + 8 * g + 4 * hh;
                uint2 w;
                w.x = pack2<T>(o[db][4 * g] * inv, o[db][4 * g + 1] * inv);
                w.y = pack2<T>(o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv);
                *reinterpret_cast<uint2*>(orow + d) = w;
            }
        }
        if (hh == 0) lse_base[row] = lt > 0.0f ? (m + fast_log2(lt)) * kLn2 : INFINITY;
    }
}

// ---------------------------------------------------------------------------
// Ping-pong forward (plain scaled dot product, head size 128, dense grid with
// no mask or dropout): 8 waves, 256 query rows per block, one block per CU.
// Waves 0-3 and 4-7 form two groups on the same four SIMDs (wave w runs on
// SIMD w % 4). Every slot of the loop ends at a block barrier; in each slot one
// group runs its MFMA phase (O^T += V^T P^T of the previous tile, then
// S^T = K Q^T of the current one) while the other runs its softmax phase
// (row max, exp2, row sum, P^T packing). One group trails the other by a slot,
// so on every SIMD the matrix core and the VALU serve different waves at the
// same time instead of both waves reaching the same phase together.
//
// What bounds it: an MFMA phase reads 32 KB of LDS operands per wave, and with
// one reading wave per SIMD the LDS delivers about half the bandwidth it gives
// two (about 97 vs 193 B/clk/CU for 16-byte reads, measured), so the phase
// runs about 1.9k cycles for 1k cycles of MFMA. It beats the 128-row tiled
// kernel on unmasked grids (+5 %); on causal, windowed and dropout grids the
// tiled kernel wins (diagonal waste of 256-row blocks, longer softmax phases).
//
// K/V tiles of 64 keys go HBM -> LDS by direct buffer loads into a ring of 4
// stages. Tile j is read in slots 2j .. 2j + 3 (K by the MFMA phases of tile j,
// V by those of tile j + 1); its copy is issued in slot 2j - 4 and must have
// landed by the end of slot 2j - 1, so three slots hide its latency. The copies
// are issued from inline assembly: the compiler would otherwise wait for every
// copy in flight before the next LDS read.
// ---------------------------------------------------------------------------
constexpr int kPPStages = 4;


template <typename T, int D>
__global__ void __launch_bounds__(512, 1) flash_fwd_pp_kernel(const FwdParams p) {
    constexpr int NW = 8;
    constexpr int BN = kBN;
    constexpr int BM = 32 * NW;
    constexpr int KS = D / 16;
    constexpr int DB = D / 32;
    constexpr int TILE = BN * D;
    constexpr int STAGE = 2 * TILE;  // K tile, then V tile
    // Direct loads each wave issues per tile (K and V): its vmcnt share.
    constexpr int LPT = 2 * (BN * D / 512) / NW;
    static_assert(LPT > 0 && LPT < 16, "loads per tile");

    __shared__ __attribute__((aligned(1024))) uint16_t kv_lds[kPPStages * STAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar copy addresses
    // Waves 4-7 lead (measured slightly faster than waves 0-3 leading).
    const int grp = (wave >> 2) ^ 1;
    const int l32 = lane & 31;
    const int hh = lane >> 5;
    const TileOffs<D> to(lane);

    // Sequence-major order: the blocks of one (batch, KV head) run together and
    // share its K/V tiles in L2.
    const int per_seq = p.q_blocks * p.heads;
    const int b = blockIdx.x / per_seq;
    const int rem = blockIdx.x - b * per_seq;
    const int qo = rem / p.heads;
    const int idx = rem - qo * p.heads;
    const int head = (idx % p.kv_heads) * p.gqa + idx / p.kv_heads;
    const int kvh = head / p.gqa;
    const int qb = p.q_blocks - 1 - qo;
    const int sq = p.seqlen_q, sk = p.seqlen_k;
    const int row0 = qb * BM;
    if (row0 >= sq) return;

    const uint16_t* qbase = static_cast<const uint16_t*>(p.q) + b * p.q_b + head * p.q_h;
    const uint16_t* kbase = static_cast<const uint16_t*>(p.k) + b * p.k_b + kvh * p.k_h;
    const uint16_t* vbase = static_cast<const uint16_t*>(p.v) + b * p.v_b + kvh * p.v_h;
    uint16_t* obase = static_cast<uint16_t*>(p.o) + b * p.o_b + head * p.o_h;
    float* lse_base = p.lse + b * p.lse_b + head * p.lse_h;

    const int n = (sk + BN - 1) / BN;

    const int row = row0 + 32 * wave + l32;

    u32x4 qf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        qf[ks] = row < sq ? *reinterpret_cast<const u32x4*>(qbase + row * p.q_s + 16 * ks + 8 * hh)
                          : u32x4{0, 0, 0, 0};
    }
    const float c = p.scale_log2;

    f32x16 o[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db] = f32x16{};
    f32x16 sc[2] = {f32x16{}, f32x16{}};
    u32x4 pk[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) pk[tt] = u32x4{0, 0, 0, 0};
    float m = -INFINITY, l = 0.0f;

    auto copy_tile = [&](int t) __attribute__((always_inline)) {
        const int kb = t * BN;
        uint16_t* st = kv_lds + (t % kPPStages) * STAGE;
        copy_rows_dma<D, NW, BN>(kbase + static_cast<int64_t>(kb) * p.k_s, p.k_s, sk - kb, st, wave, lane);
        copy_rows_dma<D, NW, BN>(vbase + static_cast<int64_t>(kb) * p.v_s, p.v_s, sk - kb, st + TILE, wave,
                                 lane);
    };

    // MFMA phase of step t: O^T += V^T P^T for tile t - 1, then S^T = K Q^T for
    // tile t. The operand reads run kLook MFMAs ahead of their use (register
    // ring), interleaved one MFMA at a time.
    auto mphase_impl = [&](auto pv_tag, auto qk_tag, int t) __attribute__((always_inline)) {
        constexpr bool PV = decltype(pv_tag)::value;
        constexpr bool QK = decltype(qk_tag)::value;
        constexpr int NPV = PV ? 4 * DB : 0;
        constexpr int NQK = QK ? 2 * KS : 0;
        constexpr int N = NPV + NQK;
        constexpr int LOOK = 4;
        const uint16_t* vl = kv_lds + ((t + kPPStages - 1) % kPPStages) * STAGE + TILE;
        const uint16_t* kl = kv_lds + (t % kPPStages) * STAGE;
        // PV step i: tt = i / DB, db = i % DB (consecutive MFMAs use different
        // accumulators); QK step j: half j % 2, k-step j / 2.
        auto load = [&](auto ic) __attribute__((always_inline)) -> u32x4 {
            constexpr int i = decltype(ic)::value;
            if constexpr (i < NPV) {
                return to.tr(vl, i % DB, i / DB);
            } else {
                return to.rm(kl, (i - NPV) & 1, (i - NPV) >> 1);
            }
        };
        // The MFMA-phase wave takes issue priority over the softmax-phase wave
        // of its SIMD (otherwise the older wave of the pair wins arbitration
        // whichever phase it is in).
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(1);
        if constexpr (QK) {
            sc[0] = f32x16{};
            sc[1] = f32x16{};
        }
        u32x4 ring[LOOK];
        constexpr int NPRO = LOOK < N ? LOOK : N;
        static_for<0, NPRO>([&](auto ic) __attribute__((always_inline)) { ring[decltype(ic)::value] = load(ic); });
        // Reads of the first NPRO operands, then (reads of operand i + LOOK, MFMA i).
        constexpr int PRO_READS = 2 * (NPRO < NPV ? NPRO : NPV) + (NPRO > NPV ? NPRO - NPV : 0);
        __builtin_amdgcn_sched_group_barrier(0x100, PRO_READS, 0);
        static_for<0, N>([&](auto ic) __attribute__((always_inline)) {
            constexpr int i = decltype(ic)::value;
            const u32x4 a = ring[i % LOOK];
            if constexpr (i + LOOK < N) {
                ring[i % LOOK] = load(std::integral_constant<int, i + LOOK>{});
                __builtin_amdgcn_sched_group_barrier(0x100, (i + LOOK < NPV) ? 2 : 1, 0);
            }
            if constexpr (i < NPV) {
                o[i % DB] = mfma32<T>(a, pk[i / DB], o[i % DB]);
            } else {
                constexpr int j = i - NPV;
                sc[j & 1] = mfma32<T>(a, qf[j >> 1], sc[j & 1]);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        });
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
    };
    // Softmax phase of tile t: P^T packed into the B operand of the next MFMA phase.
    auto vphase = [&](int t) __attribute__((always_inline)) {
        // Only the last tile can cross the end of the keys.
        const int kb = t * BN;
        if (kb + BN > sk) {
#pragma unroll
            for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int col = kb + 32 * sub + 8 * (r >> 2) + 4 * hh + (r & 3);
                    sc[sub][r] = col >= sk ? -INFINITY : sc[sub][r];
                }
            }
        }
        float mx = lane_max32(sc[0], sc[1]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m2 = mx * c;
        if (__any(m2 > m + kRescaleSlack)) {
            const float m_new = fmaxf(m, m2);
            const float alpha = (m_new == -INFINITY) ? 1.0f : fast_exp2(m - m_new);
            m = m_new;
            l *= alpha;
#pragma unroll
            for (int db = 0; db < DB; ++db) o[db] *= alpha;
        }
        const float neg_m = (m == -INFINITY) ? 0.0f : -m;
        float rowsum = 0.0f;
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float pv = fast_exp2(__builtin_fmaf(sc[sub][r], c, neg_m));
                sc[sub][r] = pv;
                rowsum += pv;
            }
        }
        l += rowsum;
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                pk[tt][w] = pack2<T>(sc[tt >> 1][8 * (tt & 1) + 2 * w], sc[tt >> 1][8 * (tt & 1) + 2 * w + 1]);
            }
        }
    };

    // Slot s: even slots issue the copy of tile s / 2 + 2; odd slot 2k + 1 ends
    // with tile k + 1 resident (tile k + 2 may still be in flight).
    auto slot_begin = [&](int s) __attribute__((always_inline)) {
        if ((s & 1) == 0 && s / 2 + 2 < n) copy_tile(s / 2 + 2);
    };
    auto slot_end = [&](int s) __attribute__((always_inline)) {
        if (s & 1) {
            if (s / 2 + 2 < n) {
                wait_vmem_le<LPT>();
            } else {
                wait_vmem_le<0>();
            }
        }
        slot_barrier();
    };

    if (n > 0) copy_tile(0);
    if (n > 1) {
        copy_tile(1);
        wait_vmem_le<LPT>();
    } else {
        wait_vmem_le<0>();
    }
    slot_barrier();

    // The first and last MFMA phases (QK only, PV only) are peeled so the
    // steady-state loop body is one straight-line sequence per group.
    const std::true_type yes{};
    const std::false_type no{};
    if (n > 0) {
        if (grp == 0) {
            slot_begin(0);
            mphase_impl(no, yes, 0);
            slot_end(0);
            slot_begin(1);
            vphase(0);
            slot_end(1);
            for (int t = 1; t < n; ++t) {
                slot_begin(2 * t);
                mphase_impl(yes, yes, t);
                slot_end(2 * t);
                slot_begin(2 * t + 1);
                vphase(t);
                slot_end(2 * t + 1);
            }
            slot_begin(2 * n);
            mphase_impl(yes, no, n);
            slot_end(2 * n);
            slot_begin(2 * n + 1);
            slot_end(2 * n + 1);
        } else {
            slot_begin(0);
            slot_end(0);
            slot_begin(1);
            mphase_impl(no, yes, 0);
            slot_end(1);
            for (int t = 1; t < n; ++t) {
                slot_begin(2 * t);
                vphase(t - 1);
                slot_end(2 * t);
                slot_begin(2 * t + 1);
                mphase_impl(yes, yes, t);
                slot_end(2 * t + 1);
            }
            slot_begin(2 * n);
            vphase(n - 1);
            slot_end(2 * n);
            slot_begin(2 * n + 1);
            mphase_impl(yes, no, n);
            slot_end(2 * n + 1);
        }
    }

    const float lt = l + __shfl_xor(l, 32, 64);
    if (row < sq) {
        const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
        uint16_t* orow = obase + row * p.o_s;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = 32 * db + 8 * g + 4 * hh;
                uint2 w;
                w.x = pack2<T>(o[db][4 * g] * inv, o[db][4 * g + 1] * inv);
                w.y = pack2<T>(o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv);
                *reinterpret_cast<uint2*>(orow + d) = w;
            }
        }
        if (hh == 0) lse_base[row] = lt > 0.0f ? (m + fast_log2(lt)) * kLn2 : INFINITY;
    }
}

// Split-KV merge (flash-attn2-rs/src/device/varlen/merge.rs): per row,
// LSE = log sum_i exp(LSE_i) and O = sum_i exp(LSE_i - LSE) O_i over the splits;
// a row no split saw gets O = 0 and LSE = +inf, as an empty row does. One wave
// per (head, packed row); lane l < D / PER owns columns PER l .. PER l + PER - 1
// (PER = 2, or 4 at D = 256). Packed row
// t is row t % rows_per_seq of sequence t / rows_per_seq in out / lse
// (rows_per_seq = total_q with zero batch strides for packed outputs).
constexpr uint32_t kUnseenLse = 0x7FC0DEADu;  // a quiet-NaN payload no kernel computes

template <typename T, int D>
__global__ void __launch_bounds__(256) merge_splits_kernel(const float* __restrict__ o_part,
                                                           const float* __restrict__ lse_part, int n_splits,
                                                           int heads, int total_q, int rows_per_seq,
                                                           uint16_t* __restrict__ o, int64_t o_b, int64_t o_s,
                                                           int64_t o_h, float* __restrict__ lse, int64_t lse_b,
                                                           int64_t lse_h) {
    constexpr int PER = D > 128 ? 4 : 2;
    static_assert(D % PER == 0 && D / PER <= 64, "one wave covers the row");
    using Vec = std::conditional_t<PER == 4, float4, float2>;
    const int lane = threadIdx.x & 63;
    const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (item >= static_cast<int64_t>(heads) * total_q) return;
    const int head = static_cast<int>(item / total_q);
    const int row = static_cast<int>(item - static_cast<int64_t>(head) * total_q);
    const int64_t stride = static_cast<int64_t>(heads) * total_q;  // between splits
    // Rows of no valid sequence keep the caller's output (plain varlen calls
    // pre-fill the partial LSE with this payload; every block of a valid
    // sequence overwrites it).
    if (__float_as_uint(lse_part[item]) == kUnseenLse) return;
    // Lane i holds the LSE of splits i and i + 64 (n_splits <= 128): one load
    // each, wave reductions for the max and the sum, then the O rows of the
    // splits eight at a time with their loads issued together.
    const float l0 = lane < n_splits ? lse_part[lane * stride + item] : -INFINITY;
    const float l1 = lane + 64 < n_splits ? lse_part[(lane + 64) * stride + item] : -INFINITY;
    float mx = fmaxf(l0, l1);
#pragma unroll
    for (int sh = 32; sh > 0; sh >>= 1) mx = fmaxf(mx, __shfl_xor(mx, sh, 64));
    float acc[PER] = {};
    float out_lse = INFINITY;
    if (mx > -INFINITY) {
        float sum = expf(l0 - mx) + expf(l1 - mx);
#pragma unroll
        for (int sh = 32; sh > 0; sh >>= 1) sum += __shfl_xor(sum, sh, 64);
        out_lse = mx + logf(sum);
        const float w0 = expf(l0 - out_lse), w1 = expf(l1 - out_lse);
        const int col = PER * (lane < D / PER ? lane : 0);
        for (int i0 = 0; i0 < n_splits; i0 += 8) {
            float w[8];
            Vec v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int i = i0 + u;
                w[u] = i < 64 ? __shfl(w0, i & 63, 64) : __shfl(w1, i & 63, 64);
                // A split that saw no key of the row has weight 0 and may hold
                // no partial row at all: its values are never used.
                v[u] = (i < n_splits && w[u] != 0.0f)
                           ? *reinterpret_cast<const Vec*>(o_part + (i * stride + item) * D + col)
                           : Vec{};
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (i0 + u < n_splits && w[u] != 0.0f) {
                    acc[0] += w[u] * v[u].x;
                    acc[1] += w[u] * v[u].y;
                    if constexpr (PER == 4) {
                        acc[2] += w[u] * v[u].z;
                        acc[3] += w[u] * v[u].w;
                    }
                }
            }
        }
    }
    const int seq = row / rows_per_seq;
    const int r = row - seq * rows_per_seq;
    if (lane < D / PER) {
        uint16_t* dst =
            o + seq * o_b + static_cast<int64_t>(r) * o_s + static_cast<int64_t>(head) * o_h + PER * lane;
        if constexpr (PER == 4) {
            *reinterpret_cast<uint2*>(dst) = uint2{pack2<T>(acc[0], acc[1]), pack2<T>(acc[2], acc[3])};
        } else {
            *reinterpret_cast<uint32_t*>(dst) = pack2<T>(acc[0], acc[1]);
        }
    }
    if (lane == 0) lse[seq * lse_b + static_cast<int64_t>(head) * lse_h + r] = out_lse;
}

// Empty-key rows: O = 0, LSE = +inf (host/forward/mod.rs:548-572). Also clears
// the output when zero_tensors is requested. Uses kernels rather than
// hipMemsetAsync so the calls stay safe inside captured graphs.
__global__ void fill_rows_kernel(uint16_t* o, int64_t o_rows, int64_t row_stride_tokens,
                                 int64_t row_elems, int64_t o_row_stride) {
    (void)row_stride_tokens;
    const int64_t total = o_rows * row_elems;
    for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < total; i += gridDim.x * 256ll) {
        const int64_t r = i / row_elems;
        const int64_t c = i - r * row_elems;
        o[r * o_row_stride + c] = 0;
    }
}

__global__ void fill_f32_kernel(float* x, int64_t n, float value) {
    for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += gridDim.x * 256ll) x[i] = value;
}

}  // namespace attn

namespace {

using namespace attn;

void fill_f32(float* x, int64_t n, float value, hipStream_t s) {
    if (n <= 0) return;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 65536);
    fill_f32_kernel<<<static_cast<unsigned>(blocks), 256, 0, s>>>(x, n, value);
    check_launch("fill lse");
}

// Zeroes a [rows, cols] view of 16-bit elements with a given row stride.
void zero_rows(void* o, int64_t rows, int64_t cols, int64_t row_stride, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return;
    const int64_t blocks = std::min<int64_t>((rows * cols + 255) / 256, 65536);
    fill_rows_kernel<<<static_cast<unsigned>(blocks), 256, 0, s>>>(static_cast<uint16_t*>(o), rows,
                                                                  0, cols, row_stride);
    check_launch("zero output");
}

struct Config {
    int qt;
    int nw;
};

// Tile configuration per head-dim bucket.
Config config_for(int D) {
    (void)D;
    return Config{1, 4};
}

template <typename T, int D, int QT, int NW, bool VARLEN>
void launch_cfg(FwdParams& prm, bool general, hipStream_t s) {
    constexpr int BM = 32 * QT * NW;
    prm.q_blocks = (prm.seqlen_q + BM - 1) / BM;
    const int64_t blocks = static_cast<int64_t>(prm.q_blocks) * prm.batch * prm.heads;
    if (blocks == 0) return;
    if (blocks > INT32_MAX) throw value_error("attention grid exceeds the launch limit");
    prm.xcd_groups = ((static_cast<int64_t>(prm.batch) * prm.kv_heads) % 8 == 0) ? 1 : 0;
    if (general) {
        flash_fwd_kernel<T, D, QT, NW, VARLEN, true><<<static_cast<unsigned>(blocks), NW * 64, 0, s>>>(prm);
    } else {
        flash_fwd_kernel<T, D, QT, NW, VARLEN, false><<<static_cast<unsigned>(blocks), NW * 64, 0, s>>>(prm);
    }
    check_launch("launch flash_fwd");
}

template <typename T, int D, bool VARLEN>
void launch_tiled(FwdParams& prm, hipStream_t s) {
    constexpr int BM = 128;
    prm.q_blocks = (prm.seqlen_q + BM - 1) / BM;
    const int64_t blocks = static_cast<int64_t>(prm.q_blocks) * prm.batch * prm.heads *
                           (prm.n_splits > 1 ? prm.n_splits : 1);
    if (blocks == 0) return;
    if (blocks > INT32_MAX) throw value_error("attention grid exceeds the launch limit");
    prm.xcd_groups = ((static_cast<int64_t>(prm.batch) * prm.kv_heads) % 8 == 0) ? 1 : 0;
    // Sequence-major order for packed sequences and unmasked grids (blocks of
    // equal work); masked dense grids keep the longest-first tile-major order.
    prm.seq_major = (VARLEN || (prm.window_left < 0 && prm.window_right < 0)) ? 1 : 0;
    if (prm.scored) {
        if (prm.drop_threshold < 255) {
            flash_fwd_tiled_kernel<T, D, VARLEN, true, false, true><<<static_cast<unsigned>(blocks), 256, 0, s>>>(prm);
        } else {
            flash_fwd_tiled_kernel<T, D, VARLEN, false, false, true><<<static_cast<unsigned>(blocks), 256, 0, s>>>(prm);
        }
    } else if (prm.drop_threshold < 255) {
        flash_fwd_tiled_kernel<T, D, VARLEN, true, false><<<static_cast<unsigned>(blocks), 256, 0, s>>>(prm);
    } else if constexpr (VARLEN) {
        if (prm.cache_mode && prm.q_blocks == 1 && prm.heads == prm.kv_heads) {
            // One query tile per sequence and one query head per KV head (e.g.
            // grouped decode rows): each K/V tile is read by one block only.
            flash_fwd_tiled_kernel<T, D, true, false, true><<<static_cast<unsigned>(blocks), 256, 0, s>>>(prm);
        } else {
            flash_fwd_tiled_kernel<T, D, true, false, false><<<static_cast<unsigned>(blocks), 256, 0, s>>>(prm);
        }
    } else {
        flash_fwd_tiled_kernel<T, D, false, false, false><<<static_cast<unsigned>(blocks), 256, 0, s>>>(prm);
    }
    check_launch("launch flash_fwd");
}

template <typename T, int D, bool VARLEN>
void launch_pp(FwdParams& prm, hipStream_t s) {
    constexpr int BM = 256;
    prm.q_blocks = (prm.seqlen_q + BM - 1) / BM;
    const int64_t blocks = static_cast<int64_t>(prm.q_blocks) * prm.batch * prm.heads;
    if (blocks == 0) return;
    if (blocks > INT32_MAX) throw value_error("attention grid exceeds the launch limit");
    prm.xcd_groups = ((static_cast<int64_t>(prm.batch) * prm.kv_heads) % 8 == 0) ? 1 : 0;
    prm.seq_major = 1;
    flash_fwd_pp_kernel<T, D><<<static_cast<unsigned>(blocks), 512, 0, s>>>(prm);
    check_launch("launch flash_fwd");
}

template <typename T, int D, bool VARLEN>
void launch_d(FwdParams& prm, bool general, hipStream_t s) {
    if constexpr (D == 64 || D == 128 || D == 256) {
        if (!general) {
            // Dense unmasked D = 128 without dropout: the ping-pong kernel
            // (measured faster there; the 128-row tiled kernel wins on causal,
            // windowed, dropout, packed and D = 64 grids).
            if constexpr (D == 128 && !VARLEN) {
                if (prm.window_left < 0 && prm.window_right < 0 && prm.drop_threshold == 255 &&
                    prm.n_splits <= 1 && !prm.scored) {
                    return launch_pp<T, D, VARLEN>(prm, s);
                }
            }
            return launch_tiled<T, D, VARLEN>(prm, s);
        }
    }
    launch_cfg<T, D, 1, 4, VARLEN>(prm, general, s);
}

template <bool VARLEN>
void launch_fwd(FwdParams& prm, int dtype, int bucket, bool general, hipStream_t s) {
    auto by_d = [&](auto tag) {
        using T = decltype(tag);
        switch (bucket) {
            case 32: launch_d<T, 32, VARLEN>(prm, general, s); break;
            case 64: launch_d<T, 64, VARLEN>(prm, general, s); break;
            case 96: launch_d<T, 96, VARLEN>(prm, general, s); break;
            case 128: launch_d<T, 128, VARLEN>(prm, general, s); break;
            case 160: launch_d<T, 160, VARLEN>(prm, general, s); break;
            case 192: launch_d<T, 192, VARLEN>(prm, general, s); break;
            case 224: launch_d<T, 224, VARLEN>(prm, general, s); break;
            case 256: launch_d<T, 256, VARLEN>(prm, general, s); break;
            default: throw value_error("unsupported head dim bucket " + std::to_string(bucket));
        }
    };
    if (dtype == KCR_BFLOAT16) {
        by_d(bf16_t{});
    } else {
        by_d(f16_t{});
    }
}

int bucket_for(int64_t d) { return static_cast<int>((d + 31) / 32 * 32); }

void check_alibi(const kcr_tensor* alibi, int64_t b, int64_t h, int32_t& alibi_b) {
    alibi_b = 0;
    if (!alibi) return;
    if (alibi->dtype != KCR_FLOAT32) throw type_error("alibi_slopes must be float32");
    if (!is_contiguous(*alibi)) throw value_error("alibi_slopes must be contiguous");
    if (alibi->ndim == 1 && alibi->shape[0] == h) {
        alibi_b = 0;
    } else if (alibi->ndim == 2 && alibi->shape[0] == b && alibi->shape[1] == h) {
        alibi_b = static_cast<int32_t>(h);
    } else {
        throw value_error("alibi_slopes must be [" + std::to_string(h) + "] or [" +
                          std::to_string(b) + ", " + std::to_string(h) + "]");
    }
    require_device(alibi, "alibi_slopes");
}

// The tile loads bound each K/V tile by its row count: rows must not overlap
// (sequence stride >= head size) and 64 rows must span less than 2 GiB.
void check_kv_rows(const kcr_tensor* k, const kcr_tensor* v, int seq_dim, int64_t d) {
    for (auto* t : {k, v}) {
        const int64_t s = t->strides[seq_dim];
        if (t->shape[seq_dim] > 1 && (s < d || s > (int64_t{1} << 23))) {
            throw value_error("k and v rows must not overlap (sequence stride >= head size) and the "
                              "sequence stride must be at most 2^23 elements");
        }
    }
}

void check_head_dim(int64_t d) {
    if (d > 256) throw value_error("head dim must be <= 256, got " + std::to_string(d));
    if (d < 8 || d % 8 != 0) {
        throw value_error("head_size must be a positive multiple of 8 (like the reference), got " +
                          std::to_string(d));
    }
}

}  // namespace
}  // namespace kcr

using namespace kcr;
using namespace kcr::attn;

namespace {
// The dense forward launch over tensors the kernels accept as they are.
void run_dense_fwd(const kcr_tensor* q, const kcr_tensor* k, const kcr_tensor* v, const kcr_tensor* alibi,
                   int32_t alibi_b, const Options& opt, const DropoutArgs& drop, int64_t B, int64_t Sq,
                   int64_t H, int64_t D, int64_t Sk, int64_t Hk, const kcr_tensor* out,
                   const kcr_tensor* lse, const kcr_tensor* probs, hipStream_t s);

int64_t round128(int64_t n) { return (n + 127) / 128 * 128; }

// Head size the forward kernels run at. Head sizes below 128 that are not a
// multiple of 32 run on the tiled kernels through zero-padded copies, 64 or
// 128 wide (the zero columns add nothing to Q K^T, and O's first D columns are
// copied back): the general kernel runs them at a rounded-up width with
// per-column masks (D = 48 236 -> 326, D = 112 341 -> 490 TFLOP/s padded).
// Multiples of 32 keep their own size below 128: the general kernel at D = 96
// (579 TFLOP/s) beats the padded D = 128 tiles (444). Above 128 the D = 256
// tiles (~975 TFLOP/s causal at 256) beat the general kernel with the
// padding's extra work and copies (causal: D = 136 250 -> 455, D = 160 503 ->
// 541, D = 192 535 -> 634).
int64_t fwd_work_dim(int64_t D) {
    if (D > 128 && D < 256 && D % 8 == 0) return 256;
    if (D % 8 != 0 || D % 32 == 0 || D > 128) return D;
    return D < 64 ? 64 : 128;
}

// The diagnostic-probability output of a forward with return_softmax
// (host/forward/mod.rs:181-199, 382-398; host/varlen/mod.rs:201-209, 400-414):
// dropout with an RNG-state tensor, and a contiguous [batch, H, ceil128(Sq),
// ceil128(Sk)] tensor of q's dtype.
void check_probabilities(const kcr_tensor* probs, const kcr_dropout* dropout, const DropoutArgs& drop,
                         const kcr_tensor* q, int64_t batch, int64_t H, int64_t Sq, int64_t Sk) {
    if (drop.threshold >= 255 || !dropout || !dropout->rng_state) {
        throw value_error("return_softmax requires nonzero dropout and a CUDA RNG-state tensor");
    }
    if (!probs || probs->dtype != q->dtype || probs->ndim != 4 || probs->shape[0] != batch ||
        probs->shape[1] != H || probs->shape[2] != round128(Sq) || probs->shape[3] != round128(Sk) ||
        !is_contiguous(*probs) || reinterpret_cast<uintptr_t>(probs->data) % 8 != 0) {
        throw value_error("probabilities must be a contiguous tensor of q's dtype with shape [" +
                          std::to_string(batch) + ", " + std::to_string(H) + ", " +
                          std::to_string(round128(Sq)) + ", " + std::to_string(round128(Sk)) + "]");
    }
    require_device(probs, "probabilities");
}

void dense_fwd_impl(const kcr_tensor* q, const kcr_tensor* k, const kcr_tensor* v, const kcr_tensor* alibi,
                    int has_scale, double scale, int causal, int64_t window_left, int64_t window_right,
                    double softcap, const kcr_dropout* dropout, const kcr_tensor* out, const kcr_tensor* lse,
                    const kcr_tensor* probs, void* stream) {
    {
        check_qkv(q, "q", 4);
        check_qkv(k, "k", 4);
        check_qkv(v, "v", 4);
        if (k->dtype != q->dtype || v->dtype != q->dtype) {
            throw type_error("q, k, v must share dtype (all f16 or all bf16)");
        }
        const int64_t B = q->shape[0], Sq = q->shape[1], H = q->shape[2], D = q->shape[3];
        const int64_t Sk = k->shape[1], Hk = k->shape[2];
        if (k->shape[0] != B || k->shape[3] != D) {
            throw value_error("k must be [B, Sk, Hk, D] with q's batch and head dim");
        }
        if (shape_of(*v) != shape_of(*k)) throw value_error("v must have k's shape [B, Sk, Hk, D]");
        check_head_dim(D);
        if (Hk <= 0 || H % Hk != 0) {
            throw value_error("num_heads (" + std::to_string(H) + ") must be a multiple of num_heads_k (" +
                              std::to_string(Hk) + ")");
        }
        if (B <= 0 || H <= 0 || B > 65535 || H > 65535) {
            throw value_error("batch and heads must each be in 1..=65535, got " + std::to_string(B) +
                              " and " + std::to_string(H));
        }
        if (Sq > INT32_MAX - 256 || Sk > INT32_MAX - 256) {
            throw value_error("sequence lengths must fit int32");
        }
        int32_t alibi_b = 0;
        check_alibi(alibi, B, H, alibi_b);
        if (!out || shape_of(*out) != shape_of(*q) || out->dtype != q->dtype) {
            throw value_error("out must match q's shape, dtype and device");
        }
        if (out->strides[3] != 1 || !nonoverlapping_layout(out)) {
            throw value_error("out must have unit last stride and nonoverlapping non-negative strides; unsupported "
                              "writable layout: elements overlap or the bounded safety checks cannot prove they "
                              "are disjoint. Use a separately allocated contiguous output.");
        }
        if (!lse || lse->dtype != KCR_FLOAT32 || lse->ndim != 3 || lse->shape[0] != B ||
            lse->shape[1] != H || lse->shape[2] != Sq || !is_contiguous(*lse)) {
            throw value_error("lse must be contiguous float32 [B, H, Sq]");
        }
        require_device(q, "q");
        require_device(k, "k");
        require_device(v, "v");
        require_device(out, "out");
        require_device(lse, "lse");
        auto s = static_cast<hipStream_t>(stream);
        const Options opt = normalize_options(has_scale, scale, causal, window_left, window_right,
                                              softcap, D, Sk);
        const DropoutArgs drop = parse_dropout(dropout, softcap, q);
        if (probs) check_probabilities(probs, dropout, drop, q, B, H, Sq, Sk);
        if (Sq == 0) return;
        // Packed copies of inputs the tile loads cannot read, and of an output
        // they cannot write or that overlaps an input (host/layout.rs:46-125,
        // host/forward/mod.rs:349-376).
        Staged sq_(q, s, true), sk_(k, s, true, 1, D), sv_(v, s, true, 1, D);
        Staged so_(out, s, false, -1, 0, {q, k, v});
        q = sq_.get();
        k = sk_.get();
        v = sv_.get();
        out = so_.get();
        const int64_t DW = fwd_work_dim(D);
        const bool pad = DW != D;
        Padded pq(pad ? q : nullptr, DW, s, true), pk(pad ? k : nullptr, DW, s, true),
            pv(pad ? v : nullptr, DW, s, true), po(pad ? out : nullptr, DW, s, false);
        if (pad) {
            q = pq.get();
            k = pk.get();
            v = pv.get();
            out = po.get();
        }
        run_dense_fwd(q, k, v, alibi, alibi_b, opt, drop, B, Sq, H, DW, Sk, Hk, out, lse, probs, s);
        po.copy_out();
        so_.copy_out();
    }
}
}  // namespace

extern "C" int kcr_flash_fwd(const kcr_tensor* q, const kcr_tensor* k, const kcr_tensor* v,
                             const kcr_tensor* alibi, int has_scale, double scale, int causal,
                             int64_t window_left, int64_t window_right, double softcap, const kcr_dropout* dropout,
                             const kcr_tensor* out, const kcr_tensor* lse, void* stream) {
    return guarded([&] {
        dense_fwd_impl(q, k, v, alibi, has_scale, scale, causal, window_left, window_right, softcap, dropout,
                       out, lse, nullptr, stream);
    });
}

extern "C" int kcr_flash_fwd_softmax(const kcr_tensor* q, const kcr_tensor* k, const kcr_tensor* v,
                                     const kcr_tensor* alibi, int has_scale, double scale, int causal,
                                     int64_t window_left, int64_t window_right, double softcap,
                                     const kcr_dropout* dropout, const kcr_tensor* out, const kcr_tensor* lse,
                                     const kcr_tensor* probabilities, void* stream) {
    return guarded([&] {
        if (!probabilities) throw value_error("probabilities is required");
        dense_fwd_impl(q, k, v, alibi, has_scale, scale, causal, window_left, window_right, softcap, dropout,
                       out, lse, probabilities, stream);
    });
}

namespace {

// Merges the split partials of `prm` into its output and LSE; `rows` is the
// packed-row count per batch entry (Sq for dense calls, Tq for packed ones).
void launch_merge(const FwdParams& prm, int dtype, int bucket, int rows, hipStream_t s) {
    const unsigned grid = static_cast<unsigned>((static_cast<int64_t>(prm.heads) * prm.total_q + 3) / 4);
    auto merge = [&](auto tag) {
        using T = decltype(tag);
        if (bucket == 64) {
            merge_splits_kernel<T, 64><<<grid, 256, 0, s>>>(
                prm.o_part, prm.lse_part, prm.n_splits, prm.heads, prm.total_q, rows,
                static_cast<uint16_t*>(prm.o), prm.o_b, prm.o_s, prm.o_h, prm.lse, prm.lse_b, prm.lse_h);
        } else if (bucket == 256) {
            merge_splits_kernel<T, 256><<<grid, 256, 0, s>>>(
                prm.o_part, prm.lse_part, prm.n_splits, prm.heads, prm.total_q, rows,
                static_cast<uint16_t*>(prm.o), prm.o_b, prm.o_s, prm.o_h, prm.lse, prm.lse_b, prm.lse_h);
        } else {
            merge_splits_kernel<T, 128><<<grid, 256, 0, s>>>(
                prm.o_part, prm.lse_part, prm.n_splits, prm.heads, prm.total_q, rows,
                static_cast<uint16_t*>(prm.o), prm.o_b, prm.o_s, prm.o_h, prm.lse, prm.lse_b, prm.lse_h);
        }
    };
    if (dtype == KCR_BFLOAT16) {
        merge(bf16_t{});
    } else {
        merge(f16_t{});
    }
    check_launch("launch merge_splits");
}

// Key splits for a dense call whose query tiles cannot fill the chip: enough
// splits for about two blocks per CU (the tiled kernel runs two per CU, one at
// D = 256), each
// split at least 256 keys, at most 32 (the reference's bounds,
// host/forward/dispatch.rs:166-181). 1 means no split.
int64_t dense_splits(int64_t B, int64_t H, int64_t Sq, int64_t Sk, int cus) {
    const int64_t blocks = (Sq + 127) / 128 * B * H;
    if (Sk < 1024 || blocks >= cus || Sq * B * H > (int64_t{1} << 24)) return 1;
    const int64_t want = (2 * cus + blocks - 1) / blocks;
    return std::max<int64_t>(1, std::min<int64_t>({want, Sk / 256, 32}));
}

void run_dense_fwd(const kcr_tensor* q, const kcr_tensor* k, const kcr_tensor* v, const kcr_tensor* alibi,
                   int32_t alibi_b, const Options& opt, const DropoutArgs& drop, int64_t B, int64_t Sq,
                   int64_t H, int64_t D, int64_t Sk, int64_t Hk, const kcr_tensor* out,
                   const kcr_tensor* lse, const kcr_tensor* probs, hipStream_t s) {
    {
        if (Sk == 0) {
            // Every row is empty: O = 0, LSE = +inf.
            for (int64_t bi = 0; bi < B; ++bi) {
                auto* base = static_cast<uint16_t*>(out->data) + bi * out->strides[0];
                for (int64_t hi = 0; hi < H; ++hi) {
                    zero_rows(base + hi * out->strides[2], Sq, D, out->strides[1], s);
                }
            }
            fill_f32(static_cast<float*>(lse->data), B * H * Sq, INFINITY, s);
            return;
        }
        FwdParams prm{};
        prm.q = q->data;
        prm.k = k->data;
        prm.v = v->data;
        prm.o = out->data;
        prm.lse = static_cast<float*>(lse->data);
        prm.alibi = alibi ? static_cast<const float*>(alibi->data) : nullptr;
        prm.q_b = q->strides[0]; prm.q_s = q->strides[1]; prm.q_h = q->strides[2];
        prm.k_b = k->strides[0]; prm.k_s = k->strides[1]; prm.k_h = k->strides[2];
        prm.v_b = v->strides[0]; prm.v_s = v->strides[1]; prm.v_h = v->strides[2];
        prm.o_b = out->strides[0]; prm.o_s = out->strides[1]; prm.o_h = out->strides[2];
        prm.lse_b = H * Sq;
        prm.lse_h = Sq;
        prm.batch = static_cast<int32_t>(B);
        prm.heads = static_cast<int32_t>(H);
        prm.kv_heads = static_cast<int32_t>(Hk);
        prm.gqa = static_cast<int32_t>(H / Hk);
        prm.seqlen_q = static_cast<int32_t>(Sq);
        prm.seqlen_k = static_cast<int32_t>(Sk);
        prm.head_dim = static_cast<int32_t>(D);
        prm.window_left = opt.window_left;
        prm.window_right = opt.window_right;
        prm.alibi_b = alibi_b;
        prm.alibi_causal = opt.alibi_causal;
        prm.scale_log2 = opt.scale * kLog2e;
        prm.tanh_scale = opt.tanh_scale;
        prm.scale_eff_log2 = opt.scale_eff * kLog2e;
        set_dropout(prm, drop);
        // Softcap / ALiBi run in the tiled kernels' scored variant; head sizes
        // the tiles do not cover and non-positive plain scales take the general
        // kernel.
        prm.scored = (opt.tanh_scale > 0.0f || alibi != nullptr) ? 1 : 0;
        const bool general = D % 32 != 0 || (D != 64 && D != 128 && D != 256 && prm.scored) ||
                             (!prm.scored && !(opt.scale > 0.0f));
        const int bucket = bucket_for(D);
        const int64_t splits = (general || prm.scored || (bucket != 64 && bucket != 128 && bucket != 256) || prm.drop_threshold < 255)
                                   ? 1
                                   : dense_splits(B, H, Sq, Sk, compute_units());
        // The probabilities read the final LSE (after any merge).
        auto probabilities = [&] {
            if (probs) launch_dropout_probabilities(prm, false, q->dtype, probs->data, round128(Sq), round128(Sk), s);
        };
        if (splits <= 1) {
            launch_fwd<false>(prm, q->dtype, bucket, general, s);
            probabilities();
            return;
        }
        // Key splits for an underfilled grid (host/forward/dispatch.rs:127-238
        // plans the same trade): fp32 partials [splits, H, B * Sq, D] and
        // [splits, H, B * Sq] from the stream-ordered allocator, then the merge.
        const int64_t rows = B * Sq;
        const int64_t bytes = splits * H * rows * (bucket + 1) * static_cast<int64_t>(sizeof(float));
        void* ws = nullptr;
        check_hip(hipMallocAsync(&ws, static_cast<size_t>(bytes), s), "hipMallocAsync (split partials)");
        prm.n_splits = static_cast<int32_t>(splits);
        prm.total_q = static_cast<int32_t>(rows);
        prm.o_part = static_cast<float*>(ws);
        prm.lse_part = prm.o_part + splits * H * rows * bucket;
        launch_fwd<false>(prm, q->dtype, bucket, false, s);
        launch_merge(prm, q->dtype, bucket, static_cast<int>(Sq), s);
        check_hip(hipFreeAsync(ws, s), "hipFreeAsync (split partials)");
        probabilities();
    }
}

}  // namespace

namespace {
void varlen_fwd_impl(const kcr_tensor* q, const kcr_tensor* k, const kcr_tensor* v,
                     const kcr_tensor* cu_seqlens_q, const kcr_tensor* cu_seqlens_k, const kcr_tensor* seqused_k,
                     const kcr_tensor* leftpad_k, const kcr_tensor* alibi, int has_scale, double scale, int causal,
                     int64_t window_left, int64_t window_right, double softcap, const kcr_dropout* dropout,
                     int64_t max_seqlen_q, int64_t max_seqlen_k, int zero_tensors, const kcr_tensor* out,
                     const kcr_tensor* lse, const kcr_tensor* probs, void* stream) {
    {
        check_qkv(q, "q", 3);
        check_qkv(k, "k", 3);
        check_qkv(v, "v", 3);
        if (k->dtype != q->dtype || v->dtype != q->dtype || shape_of(*k) != shape_of(*v) ||
            k->shape[2] != q->shape[2]) {
            throw value_error("inconsistent packed attention inputs");
        }
        if (!cu_seqlens_q || cu_seqlens_q->ndim != 1 || cu_seqlens_q->shape[0] < 2) {
            throw value_error("cu_seqlens_q must have shape [batch + 1]");
        }
        const int64_t batch = cu_seqlens_q->shape[0] - 1;
        const int64_t Tq = q->shape[0], H = q->shape[1], D = q->shape[2];
        const int64_t Tk = k->shape[0], Hk = k->shape[1];
        check_head_dim(D);
        if (batch <= 0 || H <= 0 || Hk <= 0 || H % Hk != 0 || batch > 65535 || H > 65535 ||
            Tq > INT32_MAX || Tk > INT32_MAX || max_seqlen_q < 0 || max_seqlen_k < 0 ||
            max_seqlen_q > INT32_MAX - 256 || max_seqlen_k > INT32_MAX - 256) {
            throw value_error("unsupported packed attention dimensions");
        }
        auto check_meta = [&](const kcr_tensor* t, int64_t n, const char* name) {
            if (!t) return;
            if (t->dtype != KCR_INT32 || t->ndim != 1 || t->shape[0] != n || !is_contiguous(*t)) {
                throw value_error(std::string(name) + " must be contiguous int32 [" + std::to_string(n) + "]");
            }
            require_device(t, name);
        };
        if (!cu_seqlens_k) throw value_error("cu_seqlens_k is required");
        check_meta(cu_seqlens_q, batch + 1, "cu_seqlens_q");
        check_meta(cu_seqlens_k, batch + 1, "cu_seqlens_k");
        check_meta(seqused_k, batch, "seqused_k");
        check_meta(leftpad_k, batch, "leftpad_k");
        int32_t alibi_b = 0;
        check_alibi(alibi, batch, H, alibi_b);
        if (!out || shape_of(*out) != shape_of(*q) || out->dtype != q->dtype || out->strides[2] != 1) {
            throw value_error("out must match q's shape and dtype with unit last stride");
        }
        if (!lse || lse->dtype != KCR_FLOAT32 || lse->ndim != 2 || lse->shape[0] != H ||
            lse->shape[1] != Tq || !is_contiguous(*lse)) {
            throw value_error("lse must be contiguous float32 [H, total_q]");
        }
        require_device(q, "q");
        require_device(k, "k");
        require_device(v, "v");
        require_device(out, "out");
        require_device(lse, "lse");
        auto s = static_cast<hipStream_t>(stream);
        // varlen/mod.rs:250-268: single-query packs drop causality; windows use max_k.
        int causal_eff = causal;
        if (max_seqlen_q == 1 && !alibi) causal_eff = 0;
        const Options opt = normalize_options(has_scale, scale, causal_eff, window_left, window_right,
                                              softcap, D, max_seqlen_k);
        const DropoutArgs drop = parse_dropout(dropout, softcap, q);
        if (probs) check_probabilities(probs, dropout, drop, q, batch, H, max_seqlen_q, max_seqlen_k);
        // Packed copies of what the tile loads cannot use (host/layout.rs:46-125).
        Staged sq_(q, s, true), sk_(k, s, true, 0, D), sv_(v, s, true, 0, D);
        Staged so_(out, s, zero_tensors == 0, -1, 0, {q, k, v});
        q = sq_.get();
        k = sk_.get();
        v = sv_.get();
        out = so_.get();
        if (zero_tensors || max_seqlen_k == 0) {
            // varlen/mod.rs:418-443: cleared output, LSE -inf (+inf without keys).
            for (int64_t hi = 0; hi < H; ++hi) {
                zero_rows(static_cast<uint16_t*>(out->data) + hi * out->strides[1], Tq, D, out->strides[0], s);
            }
            fill_f32(static_cast<float*>(lse->data), H * Tq, max_seqlen_k == 0 ? INFINITY : -INFINITY, s);
        }
        if (Tq == 0 || max_seqlen_q == 0 || max_seqlen_k == 0) {
            // No sequence row: the probability plane is all zero (varlen/mod.rs:445-455).
            if (probs) {
                fill_f32(static_cast<float*>(probs->data),
                         batch * H * round128(max_seqlen_q) * round128(max_seqlen_k) / 2, 0.0f, s);
            }
            so_.copy_out();
            return;
        }
        // Zero-padded copies for the head sizes fwd_work_dim widens to 64, 128
        // or 256; the padded output starts as the caller's, so rows no
        // sequence covers come back unchanged.
        const int64_t DW = fwd_work_dim(D);
        const bool pad = DW != D;
        Padded pq(pad ? q : nullptr, DW, s, true), pk(pad ? k : nullptr, DW, s, true),
            pv(pad ? v : nullptr, DW, s, true), po(pad ? out : nullptr, DW, s, true);
        if (pad) {
            q = pq.get();
            k = pk.get();
            v = pv.get();
            out = po.get();
        }
        FwdParams prm{};
        prm.q = q->data;
        prm.k = k->data;
        prm.v = v->data;
        prm.o = out->data;
        prm.lse = static_cast<float*>(lse->data);
        prm.alibi = alibi ? static_cast<const float*>(alibi->data) : nullptr;
        prm.cu_q = static_cast<const int32_t*>(cu_seqlens_q->data);
        prm.cu_k = static_cast<const int32_t*>(cu_seqlens_k->data);
        prm.total_q = static_cast<int32_t>(Tq);
        prm.total_k = static_cast<int32_t>(Tk);
        prm.seqused_k = seqused_k ? static_cast<const int32_t*>(seqused_k->data) : nullptr;
        prm.leftpad_k = leftpad_k ? static_cast<const int32_t*>(leftpad_k->data) : nullptr;
        prm.q_s = q->strides[0]; prm.q_h = q->strides[1];
        prm.k_s = k->strides[0]; prm.k_h = k->strides[1];
        prm.v_s = v->strides[0]; prm.v_h = v->strides[1];
        prm.o_s = out->strides[0]; prm.o_h = out->strides[1];
        prm.lse_b = 0;
        prm.lse_h = Tq;
        prm.batch = static_cast<int32_t>(batch);
        prm.heads = static_cast<int32_t>(H);
        prm.kv_heads = static_cast<int32_t>(Hk);
        prm.gqa = static_cast<int32_t>(H / Hk);
        prm.seqlen_q = static_cast<int32_t>(max_seqlen_q);
        prm.seqlen_k = static_cast<int32_t>(max_seqlen_k);
        prm.head_dim = static_cast<int32_t>(DW);
        prm.window_left = opt.window_left;
        prm.window_right = opt.window_right;
        prm.alibi_b = alibi_b;
        prm.alibi_causal = opt.alibi_causal;
        prm.scale_log2 = opt.scale * kLog2e;
        prm.tanh_scale = opt.tanh_scale;
        prm.scale_eff_log2 = opt.scale_eff * kLog2e;
        set_dropout(prm, drop);
        // Softcap / ALiBi run in the tiled kernels' scored variant; head sizes
        // the tiles do not cover and non-positive plain scales take the general
        // kernel.
        prm.scored = (opt.tanh_scale > 0.0f || alibi != nullptr) ? 1 : 0;
        const bool general = DW % 32 != 0 || (DW != 64 && DW != 128 && DW != 256 && prm.scored) ||
                             (!prm.scored && !(opt.scale > 0.0f));
        const int bucket = bucket_for(DW);
        const int64_t splits = (general || prm.scored || (bucket != 64 && bucket != 128 && bucket != 256) || prm.drop_threshold < 255)
                                   ? 1
                                   : dense_splits(batch, H, max_seqlen_q, max_seqlen_k, compute_units());
        if (splits <= 1) {
            launch_fwd<true>(prm, q->dtype, bucket, general, s);
        } else {
            // Key splits for an underfilled packed grid, as for dense calls; rows
            // of no valid sequence are left as they are (see merge_splits_kernel).
            const int64_t bytes = splits * H * Tq * (bucket + 1) * static_cast<int64_t>(sizeof(float));
            void* ws = nullptr;
            check_hip(hipMallocAsync(&ws, static_cast<size_t>(bytes), s), "hipMallocAsync (split partials)");
            prm.n_splits = static_cast<int32_t>(splits);
            prm.o_part = static_cast<float*>(ws);
            prm.lse_part = prm.o_part + splits * H * Tq * bucket;
            fill_f32(prm.lse_part, H * Tq, __builtin_bit_cast(float, kUnseenLse), s);
            launch_fwd<true>(prm, q->dtype, bucket, false, s);
            launch_merge(prm, q->dtype, bucket, static_cast<int>(Tq), s);
            check_hip(hipFreeAsync(ws, s), "hipFreeAsync (split partials)");
        }
        if (probs) {
            launch_dropout_probabilities(prm, true, q->dtype, probs->data, round128(max_seqlen_q),
                                         round128(max_seqlen_k), s);
        }
        po.copy_out();
        so_.copy_out();
    }
}
}  // namespace

extern "C" int kcr_flash_varlen_fwd(const kcr_tensor* q, const kcr_tensor* k, const kcr_tensor* v,
                                    const kcr_tensor* cu_seqlens_q, const kcr_tensor* cu_seqlens_k,
                                    const kcr_tensor* seqused_k, const kcr_tensor* leftpad_k,
                                    const kcr_tensor* alibi, int has_scale, double scale,
                                    int causal, int64_t window_left, int64_t window_right,
                                    double softcap, const kcr_dropout* dropout, int64_t max_seqlen_q, int64_t max_seqlen_k,
                                    int zero_tensors, const kcr_tensor* out,
                                    const kcr_tensor* lse, void* stream) {
    return guarded([&] {
        varlen_fwd_impl(q, k, v, cu_seqlens_q, cu_seqlens_k, seqused_k, leftpad_k, alibi, has_scale, scale, causal,
                        window_left, window_right, softcap, dropout, max_seqlen_q, max_seqlen_k, zero_tensors, out,
                        lse, nullptr, stream);
    });
}

extern "C" int kcr_flash_varlen_fwd_softmax(const kcr_tensor* q, const kcr_tensor* k, const kcr_tensor* v,
                                            const kcr_tensor* cu_seqlens_q, const kcr_tensor* cu_seqlens_k,
                                            const kcr_tensor* seqused_k, const kcr_tensor* leftpad_k,
                                            const kcr_tensor* alibi, int has_scale, double scale, int causal,
                                            int64_t window_left, int64_t window_right, double softcap,
                                            const kcr_dropout* dropout, int64_t max_seqlen_q, int64_t max_seqlen_k,
                                            int zero_tensors, const kcr_tensor* out, const kcr_tensor* lse,
                                            const kcr_tensor* probabilities, void* stream) {
    return guarded([&] {
        if (!probabilities) throw value_error("probabilities is required");
        varlen_fwd_impl(q, k, v, cu_seqlens_q, cu_seqlens_k, seqused_k, leftpad_k, alibi, has_scale, scale, causal,
                        window_left, window_right, softcap, dropout, max_seqlen_q, max_seqlen_k, zero_tensors, out,
                        lse, probabilities, stream);
    });
}

// Split-KV scratch: fp32 partial O [n_splits, H, Tq, D] and LSE [n_splits, H, Tq].
extern "C" int64_t kcr_flash_fwd_kvcache_workspace_bytes(int64_t num_splits, int64_t heads, int64_t total_q,
                                                         int64_t head_dim) {
    if (num_splits <= 1 || heads <= 0 || total_q <= 0 || head_dim <= 0) return 0;
    const int64_t d = bucket_for(head_dim);
    return num_splits * heads * total_q * (d + 1) * static_cast<int64_t>(sizeof(float));
}

namespace {

// The cached-attention launch behind both kvcache entry points. `workspace`
// holds the split partials; `noalloc` names the fixed scratch of the
// allocation-free entry point in the size error.
void fwd_kvcache_impl(const kcr_tensor* q, const kcr_tensor* kcache, const kcr_tensor* vcache,
                      const kcr_tensor* cu_seqlens_q, const kcr_tensor* seqused_k, int64_t new_keys,
                      const kcr_tensor* leftpad_k, const kcr_tensor* cache_batch_idx,
                      const kcr_tensor* block_table, const kcr_tensor* alibi, int has_scale, double scale,
                      int causal, int64_t window_left, int64_t window_right, double softcap,
                      int64_t max_seqlen_q, int64_t num_splits, void* workspace, int64_t workspace_bytes,
                      bool noalloc, const kcr_tensor* out, const kcr_tensor* lse, void* stream) {
    {
        // Batched form: q/out [B, R, H, D] (any strides) and lse [B, H, R], no cu_seqlens_q.
        const bool batched = q && q->ndim == 4 && !cu_seqlens_q;
        check_qkv(q, "q", batched ? 4 : 3);
        check_qkv(kcache, "kcache", 4);
        check_qkv(vcache, "vcache", 4);
        if (kcache->dtype != q->dtype || vcache->dtype != q->dtype) {
            throw type_error("q, kcache and vcache must share dtype (all f16 or all bf16)");
        }
        if (shape_of(*kcache) != shape_of(*vcache)) throw value_error("K/V cache shapes must match");
        if (!batched && (!cu_seqlens_q || cu_seqlens_q->ndim != 1 || cu_seqlens_q->shape[0] < 2)) {
            throw value_error("cu_seqlens_q must have shape [batch + 1]");
        }
        const int64_t batch = batched ? q->shape[0] : cu_seqlens_q->shape[0] - 1;
        const int64_t R = batched ? q->shape[1] : 0;
        if (batched) {
            if (R <= 0 || R > 65535) throw value_error("batched q needs 1..65535 rows per sequence");
            max_seqlen_q = R;
        }
        const int64_t Tq = batched ? batch * R : q->shape[0];
        const int64_t H = q->shape[batched ? 2 : 1], D = q->shape[batched ? 3 : 2];
        const int64_t Bc = kcache->shape[0], S = kcache->shape[1], Hk = kcache->shape[2];
        check_head_dim(D);
        if (kcache->shape[3] != D) throw value_error("K/V cache shapes must match Q's head size");
        if (batch <= 0 || batch > 65535 || H <= 0 || H > 65535 || Hk <= 0 || H % Hk != 0 || Tq > INT32_MAX ||
            max_seqlen_q < 0 || max_seqlen_q > INT32_MAX - 256 || Bc <= 0 || S <= 0) {
            throw value_error("unsupported cached attention dimensions");
        }
        auto check_meta = [&](const kcr_tensor* t, std::vector<int64_t> shape, const char* name) {
            if (!t) return;
            if (t->dtype != KCR_INT32 || shape_of(*t) != shape || t->strides[t->ndim - 1] != 1 ||
                (t->ndim == 1 && !is_contiguous(*t))) {
                throw value_error(std::string(name) + " must be int32 " + shape_string(shape) +
                                  " with unit last stride");
            }
            require_device(t, name);
        };
        if (new_keys < 0 || new_keys > INT32_MAX) throw value_error("new_keys must be in 0..=i32::MAX");
        if (!batched) check_meta(cu_seqlens_q, {batch + 1}, "cu_seqlens_q");
        check_meta(seqused_k, {batch}, "seqused_k");
        check_meta(leftpad_k, {batch}, "leftpad_k");
        check_meta(cache_batch_idx, {batch}, "cache_batch_idx");
        int64_t capacity = S;
        if (block_table) {
            if (block_table->ndim != 2) throw value_error("block_table must be int32 [batch, max_blocks]");
            check_meta(block_table, {batch, block_table->shape[1]}, "block_table");
            if (S % 256 != 0 || leftpad_k || cache_batch_idx) {
                throw value_error("paged caches require page size divisible by 256 and no leftpad or cache_batch_idx");
            }
            capacity = S * block_table->shape[1];
            if (block_table->strides[0] < 0 || block_table->strides[0] > INT32_MAX) {
                throw value_error("block_table row stride must fit int32");
            }
        }
        if (capacity > INT32_MAX - 256 || Bc * S > INT32_MAX) throw value_error("cache/query dimensions must fit int32");
        int32_t alibi_b = 0;
        check_alibi(alibi, batch, H, alibi_b);
        if (!out || shape_of(*out) != shape_of(*q) || out->dtype != q->dtype || out->strides[out->ndim - 1] != 1) {
            throw value_error("out must match q's shape and dtype with unit last stride");
        }
        if (batched) {
            if (!lse || lse->dtype != KCR_FLOAT32 || shape_of(*lse) != std::vector<int64_t>{batch, H, R} ||
                lse->strides[2] != 1) {
                throw value_error("lse must be float32 [batch, H, rows] with unit last stride");
            }
        } else if (!lse || lse->dtype != KCR_FLOAT32 || lse->ndim != 2 || lse->shape[0] != H ||
                   lse->shape[1] != Tq || !is_contiguous(*lse)) {
            throw value_error("lse must be contiguous float32 [H, total_q]");
        }
        for (auto* t : {q, kcache, vcache, out}) {
            if (Tq > 0 && !rows_aligned16(t)) {
                throw value_error("q, caches and out must have 16-byte aligned rows (strides multiple of 8 elements)");
            }
        }
        check_kv_rows(kcache, vcache, 1, D);
        for (auto* t : {q, kcache, vcache, out, lse}) require_device(t, "tensor");
        if (num_splits < 0 || num_splits > 128) throw value_error("num_splits must be in 0..=128");
        auto s = static_cast<hipStream_t>(stream);
        const Options opt = normalize_options(has_scale, scale, causal, window_left, window_right, softcap, D,
                                              capacity);
        if (Tq == 0 || max_seqlen_q == 0) return;
        FwdParams prm{};
        prm.q = q->data;
        prm.k = kcache->data;
        prm.v = vcache->data;
        prm.o = out->data;
        prm.lse = static_cast<float*>(lse->data);
        prm.alibi = alibi ? static_cast<const float*>(alibi->data) : nullptr;
        prm.seqused_k = seqused_k ? static_cast<const int32_t*>(seqused_k->data) : nullptr;
        prm.seqused_add = static_cast<int32_t>(new_keys);
        prm.leftpad_k = leftpad_k ? static_cast<const int32_t*>(leftpad_k->data) : nullptr;
        prm.total_q = static_cast<int32_t>(Tq);
        prm.k_b = kcache->strides[0]; prm.k_s = kcache->strides[1]; prm.k_h = kcache->strides[2];
        prm.v_b = vcache->strides[0]; prm.v_s = vcache->strides[1]; prm.v_h = vcache->strides[2];
        if (batched) {
            prm.rows_per_seq = static_cast<int32_t>(R);
            prm.q_b = q->strides[0]; prm.q_s = q->strides[1]; prm.q_h = q->strides[2];
            prm.o_b = out->strides[0]; prm.o_s = out->strides[1]; prm.o_h = out->strides[2];
            prm.lse_b = lse->strides[0];
            prm.lse_h = lse->strides[1];
        } else {
            prm.cu_q = static_cast<const int32_t*>(cu_seqlens_q->data);
            prm.q_s = q->strides[0]; prm.q_h = q->strides[1];
            prm.o_s = out->strides[0]; prm.o_h = out->strides[1];
            prm.lse_b = 0;
            prm.lse_h = Tq;
        }
        const int rows = batched ? static_cast<int>(R) : static_cast<int>(Tq);
        prm.batch = static_cast<int32_t>(batch);
        prm.heads = static_cast<int32_t>(H);
        prm.kv_heads = static_cast<int32_t>(Hk);
        prm.gqa = static_cast<int32_t>(H / Hk);
        prm.seqlen_q = static_cast<int32_t>(max_seqlen_q);
        prm.seqlen_k = static_cast<int32_t>(capacity);
        prm.head_dim = static_cast<int32_t>(D);
        prm.window_left = opt.window_left;
        prm.window_right = opt.window_right;
        prm.alibi_b = alibi_b;
        prm.alibi_causal = opt.alibi_causal;
        prm.scale_log2 = opt.scale * kLog2e;
        prm.tanh_scale = opt.tanh_scale;
        prm.scale_eff_log2 = opt.scale_eff * kLog2e;
        prm.drop_threshold = 255;
        prm.inv_keep = 1.0f;
        prm.cache_mode = 1;
        prm.capacity = static_cast<int32_t>(capacity);
        prm.cache_batches = static_cast<int32_t>(Bc);
        prm.cache_idx = cache_batch_idx ? static_cast<const int32_t*>(cache_batch_idx->data) : nullptr;
        if (block_table) {
            prm.block_table = static_cast<const int32_t*>(block_table->data);
            prm.table_stride = block_table->strides[0];
            prm.table_cols = static_cast<int32_t>(block_table->shape[1]);
            prm.page_size = static_cast<int32_t>(S);
            prm.k_page = kcache->strides[0];
            prm.v_page = vcache->strides[0];
        }
        // Softcap / ALiBi run in the tiled kernels' scored instances (paged or
        // not, with key splits); other head sizes on the general kernel.
        prm.scored = (opt.tanh_scale > 0.0f || alibi != nullptr) ? 1 : 0;
        const bool general = D % 32 != 0 || (D != 64 && D != 128 && D != 256 && prm.scored) ||
                             (!prm.scored && !(opt.scale > 0.0f));
        const int bucket = bucket_for(D);
        const bool tiled = !general && (bucket == 64 || bucket == 128 || bucket == 256);
        if (block_table && !tiled) {
            throw value_error("paged caches support head size 64, 128 or 256 (and a positive scale)");
        }
        const int64_t splits = tiled ? std::max<int64_t>(1, num_splits) : 1;
        if (splits > 1) {
            const int64_t need = kcr_flash_fwd_kvcache_workspace_bytes(splits, H, Tq, D);
            if (noalloc && need > workspace_bytes) {
                throw value_error(std::to_string(splits) + " splits over " + std::to_string(H) + " heads x " +
                                  std::to_string(Tq) + " query rows need " + std::to_string(need) +
                                  " bytes of split scratch; kcr_flash_fwd_kvcache_noalloc holds at most " +
                                  std::to_string(workspace_bytes) +
                                  " (use fewer splits, or kcr_flash_fwd_kvcache with a workspace)");
            }
            if (!workspace || workspace_bytes < need) {
                throw value_error("workspace must hold " + std::to_string(need) + " bytes for " +
                                  std::to_string(splits) + " splits");
            }
            if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0) throw value_error("workspace must be 16-byte aligned");
            prm.n_splits = static_cast<int32_t>(splits);
            prm.o_part = static_cast<float*>(workspace);
            prm.lse_part = prm.o_part + splits * H * Tq * bucket;
            // Packed rows of an invalid sequence are unknown to its blocks: start
            // every partial LSE at -inf (batched blocks write their own).
            if (!batched) fill_f32(prm.lse_part, splits * H * Tq, -INFINITY, s);
        }
        launch_fwd<true>(prm, q->dtype, bucket, general, s);
        if (splits > 1) {
            const int64_t items = H * Tq;
            const unsigned grid = static_cast<unsigned>((items + 3) / 4);
            auto merge = [&](auto tag) {
                using T = decltype(tag);
                if (bucket == 64) {
                    merge_splits_kernel<T, 64><<<grid, 256, 0, s>>>(
                        prm.o_part, prm.lse_part, prm.n_splits, prm.heads, prm.total_q, rows,
                        static_cast<uint16_t*>(prm.o), prm.o_b, prm.o_s, prm.o_h, prm.lse, prm.lse_b, prm.lse_h);
                } else if (bucket == 256) {
                    merge_splits_kernel<T, 256><<<grid, 256, 0, s>>>(
                        prm.o_part, prm.lse_part, prm.n_splits, prm.heads, prm.total_q, rows,
                        static_cast<uint16_t*>(prm.o), prm.o_b, prm.o_s, prm.o_h, prm.lse, prm.lse_b, prm.lse_h);
                } else {
                    merge_splits_kernel<T, 128><<<grid, 256, 0, s>>>(
                        prm.o_part, prm.lse_part, prm.n_splits, prm.heads, prm.total_q, rows,
                        static_cast<uint16_t*>(prm.o), prm.o_b, prm.o_s, prm.o_h, prm.lse, prm.lse_b, prm.lse_h);
                }
            };
            if (q->dtype == KCR_BFLOAT16) {
                merge(bf16_t{});
            } else {
                merge(f16_t{});
            }
            check_launch("launch merge_splits");
        }
    }
}

// Split scratch of the allocation-free entry point: one copy per GPU, resident
// until the process ends. Host code reaches it only through the per-device
// address from hipGetSymbolAddress (the array's name is a host-side stand-in).
constexpr int64_t kNoAllocScratchBytes = 64ll << 20;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

// The device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept.
void* noalloc_scratch() {
    static std::mutex mu;
    static std::vector<void*> addr;
    int device = 0;
    check_hip(hipGetDevice(&device), "hipGetDevice");
    std::lock_guard<std::mutex> lock(mu);
    if (static_cast<size_t>(device) >= addr.size()) addr.resize(device + 1, nullptr);
    if (!addr[device]) {
        void* p = nullptr;
        check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        addr[device] = p;
    }
    return addr[device];
}

}  // namespace

extern "C" int kcr_flash_fwd_kvcache(const kcr_tensor* q, const kcr_tensor* kcache, const kcr_tensor* vcache,
                                     const kcr_tensor* cu_seqlens_q, const kcr_tensor* seqused_k,
                                     int64_t new_keys, const kcr_tensor* leftpad_k, const kcr_tensor* cache_batch_idx,
                                     const kcr_tensor* block_table, const kcr_tensor* alibi, int has_scale,
                                     double scale, int causal, int64_t window_left, int64_t window_right,
                                     double softcap, int64_t max_seqlen_q, int64_t num_splits, void* workspace,
                                     int64_t workspace_bytes, const kcr_tensor* out, const kcr_tensor* lse,
                                     void* stream) {
    return guarded([&] {
        fwd_kvcache_impl(q, kcache, vcache, cu_seqlens_q, seqused_k, new_keys, leftpad_k, cache_batch_idx,
                         block_table, alibi, has_scale, scale, causal, window_left, window_right, softcap,
                         max_seqlen_q, num_splits, workspace, workspace_bytes, false, out, lse, stream);
    });
}

extern "C" int64_t kcr_flash_fwd_kvcache_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int kcr_flash_fwd_kvcache_noalloc(const kcr_tensor* q, const kcr_tensor* kcache,
                                             const kcr_tensor* vcache, const kcr_tensor* cu_seqlens_q,
                                             const kcr_tensor* seqused_k, int64_t new_keys,
                                             const kcr_tensor* leftpad_k, const kcr_tensor* cache_batch_idx,
                                             const kcr_tensor* block_table, const kcr_tensor* alibi,
                                             int has_scale, double scale, int causal, int64_t window_left,
                                             int64_t window_right, double softcap, int64_t max_seqlen_q,
                                             int64_t num_splits, const kcr_tensor* out, const kcr_tensor* lse,
                                             void* stream) {
    return guarded([&] {
        void* ws = num_splits > 1 ? noalloc_scratch() : nullptr;
        fwd_kvcache_impl(q, kcache, vcache, cu_seqlens_q, seqused_k, new_keys, leftpad_k, cache_batch_idx,
                         block_table, alibi, has_scale, scale, causal, window_left, window_right, softcap,
                         max_seqlen_q, num_splits, ws, ws ? kNoAllocScratchBytes : 0, true, out, lse, stream);
    });
}
