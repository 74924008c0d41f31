// FlashAttention-2 backward on MI355X (gfx950): `bwd_preprocess`, `bwd_dq`,
// `bwd_dkv`, `bwd_all` and the packed `varlen_bwd_explicit`.
//
// Reference semantics: flash-attn2-rs/src/device/backward/reduce.rs:40-108
// (delta = rowsum(dO * O)), common.rs:121-152 (P recomputed from LSE, softcap
// derivative), dq.rs:12-469 (dQ), dkv.rs:13-245 (dK/dV with the query heads of a
// KV head summed in a fixed order), device/varlen/backward.rs:53-887 and
// host/backward.rs:14-757, host/varlen/backward.rs:15-546.
//
// MI355X design (two deterministic kernels, no atomics):
//   dK/dV kernel: a block owns 32*NW keys of one (batch, KV head); each wave keeps
//     its 32 keys' K and V rows in VGPRs as MFMA operands for the whole kernel and
//     accumulates dK^T and dV^T (one key per lane) in registers while the query
//     heads of the group and their query tiles stream through LDS. Scores are
//     formed as S = Q K^T so that P and dS come out of the accumulators already in
//     the B-operand layout of dV^T = dO^T P and dK^T = Q^T dS; Q and dO are staged
//     in LDS both row-major (A operand of S, dP) and transposed (A operand of dV,
//     dK), the transpose done by the loading threads in registers.
//   dQ kernel: the forward's structure with dO added: Q and dO stay in VGPRs,
//     K/V tiles stream through LDS (K also transposed for dQ^T = K^T dS^T), and
//     dS^T comes out of the accumulators in the B-operand layout.
#include "attention.h"

namespace kcr {
namespace attn {

struct BwdParams {
    const void* q;
    const void* k;
    const void* v;
    const void* dout;
    const float* lse;
    const float* delta;
    void* dq;
    void* dk;
    void* dv;
    const float* alibi;
    const int32_t* cu_q;
    const int32_t* cu_k;
    int64_t q_b, q_s, q_h;
    int64_t k_b, k_s, k_h;
    int64_t v_b, v_s, v_h;
    int64_t do_b, do_s, do_h;
    int64_t dq_b, dq_s, dq_h;
    int64_t dk_b, dk_s, dk_h;
    int64_t dv_b, dv_s, dv_h;
    int64_t lse_b, lse_h;      // dense [B,H,Sq]; varlen [H,Tq]
    int64_t delta_b, delta_h;  // dense [B,H,round128(Sq)]; varlen [H, Tq + 128 B]
    int32_t total_q, total_k;  // varlen: rows of q and k (bounds for cu_seqlens)
    int32_t batch, heads, kv_heads, gqa;
    int32_t seqlen_q, seqlen_k;
    int32_t head_dim;
    int32_t window_left, window_right;
    int32_t blocks_per_seq;  // key blocks (dkv) or query blocks (dq) per (batch, head)
    int32_t seq_major;       // varlen v2 kernels: sequence-major block order
    int32_t pair_tiles;      // dK/dV v2 kernel (paired instance): each block takes key tiles t and per - 1 - t
    int32_t alibi_b, alibi_causal;
    float scale_log2;
    float tanh_scale;
    float scale_eff_log2;
    float grad_scale;  // softmax scale (chain rule through raw scores) / keep
    const int64_t* rng_state;  // dropout: device [seed, offset], or null (fields below)
    uint64_t drop_seed, drop_offset;
    uint32_t drop_threshold;   // 255 = no dropout
    float inv_keep;            // dV scale: 1 / keep
};

// Sequence bounds of batch entry b (dense: the whole tensor).
struct SeqBounds {
    int sq, sk;
    int64_t q_off, k_off;  // first token of the sequence (varlen)
    int lse_row0, delta_row0;
    bool ok;
};

template <bool VARLEN>
__device__ __forceinline__ SeqBounds seq_bounds(const BwdParams& p, int b) {
    SeqBounds s{p.seqlen_q, p.seqlen_k, 0, 0, 0, 0, true};
    if constexpr (VARLEN) {
        const int qs = p.cu_q[b], qe = p.cu_q[b + 1];
        const int ks = p.cu_k[b], ke = p.cu_k[b + 1];
        if (qs < 0 || qe < qs || qe > p.total_q || ks < 0 || ke < ks || ke > p.total_k ||
            qe - qs > p.seqlen_q || ke - ks > p.seqlen_k) {
            s.ok = false;
            return s;
        }
        s.sq = qe - qs;
        s.sk = ke - ks;
        s.q_off = qs;
        s.k_off = ks;
        s.lse_row0 = qs;
        s.delta_row0 = qs + 128 * b;
    }
    return s;
}

// Score in the log2 domain (and the softcap derivative factor 1 - tanh^2).
template <bool GENERAL>
__device__ __forceinline__ float bwd_score(const BwdParams& p, float raw, int row, int col, int off,
                                           float slope_log2, float& dfac) {
    dfac = 1.0f;
    if constexpr (GENERAL) {
        float x;
        if (p.tanh_scale > 0.0f) {
            const float t = tanhf(raw * p.tanh_scale);
            dfac = 1.0f - t * t;
            x = t * p.scale_eff_log2;
        } else {
            x = raw * p.scale_log2;
        }
        if (p.alibi) {
            x += p.alibi_causal ? slope_log2 * static_cast<float>(col)
                                : -slope_log2 * fabsf(static_cast<float>(row + off - col));
        }
        return x;
    } else {
        return raw * p.scale_log2;
    }
}

// P = 2^(score - lse) of one element for the v2 kernels: the plain score with
// the scale folded into one FMA (c = scale log2 e) for SCORED = 0; the ALiBi
// bias added for SCORED = 1; the softcap (and any ALiBi bias) with its
// derivative factor in dfac for SCORED = 2.
template <int SCORED>
__device__ __forceinline__ float bwd_prob(const BwdParams& p, float raw, float c, float lse2, int row, int col,
                                          int off, float slope_log2, float& dfac) {
    if constexpr (SCORED != 0) {
        float x;
        dfac = 1.0f;
        if constexpr (SCORED == 2) {
            const float t = tanh_exp2(raw * p.tanh_scale);
            dfac = 1.0f - t * t;
            x = t * p.scale_eff_log2;
        } else {
            x = raw * p.scale_log2;
        }
        if (SCORED == 1 || p.alibi) {
            x += p.alibi_causal ? slope_log2 * static_cast<float>(col)
                                : -slope_log2 * fabsf(static_cast<float>(row + off - col));
        }
        return fast_exp2(x - lse2);
    } else {
        dfac = 1.0f;
        return fast_exp2(__builtin_fmaf(raw, c, -lse2));
    }
}

__device__ __forceinline__ bool masked_at(int row, int col, int sk, int off, int wl, int wr) {
    return (col >= sk) || (wr >= 0 && col > row + off + wr) || (wl >= 0 && col < row + off - wl);
}

// ---------------------------------------------------------------------------
// delta[b, h, s] = sum_d dout * out (reduce.rs:40-108); rows >= S are written 0.
// One group of D/8 lanes per row (each lane 16 bytes of dO and of O).
// ---------------------------------------------------------------------------
template <typename T, bool VARLEN>
__global__ void __launch_bounds__(256) bwd_preprocess_kernel(
    const uint16_t* __restrict__ dout, const uint16_t* __restrict__ out, float* __restrict__ delta,
    const int32_t* __restrict__ cu_q, int64_t do_b, int64_t do_s, int64_t do_h, int64_t o_b,
    int64_t o_s, int64_t o_h, int64_t delta_b, int64_t delta_h, int seq, int rounded, int heads,
    int head_dim, int lanes_per_row, float keep, int64_t total_q) {
    const int rows_per_block = 256 / lanes_per_row;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * rows_per_block + threadIdx.x / lanes_per_row;
    const int lane = threadIdx.x % lanes_per_row;
    // row -> (b, h, s) with s in [0, rounded)
    const int64_t s = row % rounded;
    const int64_t h = (row / rounded) % heads;
    const int64_t b = row / (static_cast<int64_t>(rounded) * heads);
    int sq = seq;
    int64_t qoff = 0;
    int64_t drow0 = 0;
    if constexpr (VARLEN) {
        const int qs = cu_q[b], qe = cu_q[b + 1];
        if (qs < 0 || qe < qs || qe > total_q || qe - qs > seq) return;
        sq = qe - qs;
        qoff = qs;
        drow0 = qs + 128 * b;
        if (s >= (sq + 127) / 128 * 128) return;
    }
    float sum = 0.0f;
    if (s < sq) {
        const uint16_t* a;
        const uint16_t* c;
        if constexpr (VARLEN) {
            a = dout + (qoff + s) * do_s + h * do_h;
            c = out + (qoff + s) * o_s + h * o_h;
        } else {
            a = dout + b * do_b + s * do_s + h * do_h;
            c = out + b * o_b + s * o_s + h * o_h;
        }
        for (int d = lane * 8; d < head_dim; d += lanes_per_row * 8) {
            // dO and O are read once: non-temporal loads.
            const u32x4 x = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a + d));
            const u32x4 y = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(c + d));
            float fx[8], fy[8];
            unpack8<T>(x, fx);
            unpack8<T>(y, fy);
#pragma unroll
            for (int e = 0; e < 8; ++e) sum += fx[e] * fy[e];
        }
    }
    for (int w = lanes_per_row / 2; w > 0; w >>= 1) sum += __shfl_xor(sum, w, 64);
    if (lane == 0) {
        if constexpr (VARLEN) {
            delta[h * delta_h + drow0 + s] = sum * keep;
        } else {
            delta[b * delta_b + h * delta_h + s] = sum * keep;
        }
    }
}

// ---------------------------------------------------------------------------
// dK / dV kernel.
// ---------------------------------------------------------------------------
template <typename T, int D, int NW, bool VARLEN, bool GENERAL>
__global__ void __launch_bounds__(NW * 64) flash_bwd_dkv_kernel(const BwdParams p) {
    constexpr int BK = 32 * NW;  // keys per block
    constexpr int BQ = 64;       // queries per tile
    constexpr int NT = NW * 64;
    constexpr int KS = D / 16;
    constexpr int DB = D / 32;
    constexpr int RSTR = D + 8;   // row-major tile stride
    constexpr int TSTR = BQ + 8;  // transposed tile stride
    constexpr int DCH = D / 8;
    constexpr int ITEMS = (BQ / 4) * DCH;  // 4 rows x 8 d per item
    constexpr int IPT = (ITEMS + NT - 1) / NT;

    __shared__ __attribute__((aligned(16))) uint16_t q_lds[BQ * RSTR];
    __shared__ __attribute__((aligned(16))) uint16_t do_lds[BQ * RSTR];
    __shared__ __attribute__((aligned(16))) uint16_t qt_lds[D * TSTR];
    __shared__ __attribute__((aligned(16))) uint16_t dot_lds[D * TSTR];
    __shared__ __attribute__((aligned(16))) float lse_lds[BQ];
    __shared__ __attribute__((aligned(16))) float dl_lds[BQ];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, hh = lane >> 5;

    const int per = p.blocks_per_seq;
    const int kbi = blockIdx.x % per;
    const int bkv = blockIdx.x / per;
    const int b = bkv / p.kv_heads;
    const int kvh = bkv - b * p.kv_heads;
    const SeqBounds sb = seq_bounds<VARLEN>(p, b);
    const DropoutState drop = p.drop_threshold < 255 ? dropout_state(p) : DropoutState{};
    if (!sb.ok) return;
    const int sq = sb.sq, sk = sb.sk;
    const int key0 = kbi * BK;
    if (key0 >= sk) return;
    const int off = sk - sq;
    const int wl = p.window_left, wr = p.window_right;

    const uint16_t* kbase = static_cast<const uint16_t*>(p.k) +
                            (VARLEN ? sb.k_off * p.k_s : b * p.k_b) + kvh * p.k_h;
    const uint16_t* vbase = static_cast<const uint16_t*>(p.v) +
                            (VARLEN ? sb.k_off * p.v_s : b * p.v_b) + kvh * p.v_h;

    // This wave's 32 keys: K and V rows as B operands of S = Q K^T and dP = dO V^T.
    const int wk0 = key0 + 32 * wave;
    const int my_key = wk0 + l32;
    u32x4 kf[KS], vf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const int d0 = 16 * ks + 8 * hh;
        if (my_key < sk && d0 < p.head_dim) {
            kf[ks] = *reinterpret_cast<const u32x4*>(kbase + my_key * p.k_s + d0);
            vf[ks] = *reinterpret_cast<const u32x4*>(vbase + my_key * p.v_s + d0);
        } else {
            kf[ks] = u32x4{0, 0, 0, 0};
            vf[ks] = u32x4{0, 0, 0, 0};
        }
    }

    f32x16 dk[DB], dv[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) {
        dk[db] = f32x16{};
        dv[db] = f32x16{};
    }

    // Query rows that can see some key of this block.
    const int key_last = min(key0 + BK, sk) - 1;
    int q_begin = 0;
    if (wr >= 0) q_begin = max(0, key0 - off - wr);
    q_begin = (q_begin / BQ) * BQ;
    int q_end = sq;
    if (wl >= 0) q_end = max(0, min(sq, key_last - off + wl + 1));

    for (int j = 0; j < p.gqa; ++j) {
        const int head = kvh * p.gqa + j;
        const uint16_t* qbase = static_cast<const uint16_t*>(p.q) +
                                (VARLEN ? sb.q_off * p.q_s : b * p.q_b) + head * p.q_h;
        const uint16_t* dobase = static_cast<const uint16_t*>(p.dout) +
                                 (VARLEN ? sb.q_off * p.do_s : b * p.do_b) + head * p.do_h;
        const float* lse_row = p.lse + (VARLEN ? 0 : b * p.lse_b) + head * p.lse_h + sb.lse_row0;
        const float* dl_row = p.delta + (VARLEN ? 0 : b * p.delta_b) + head * p.delta_h + sb.delta_row0;
        float slope_log2 = 0.0f;
        if constexpr (GENERAL) {
            if (p.alibi) slope_log2 = p.alibi[b * p.alibi_b + head] * kLog2e;
        }

        for (int qb = q_begin; qb < q_end; qb += BQ) {
            // ---- stage Q, dO (row-major and transposed), LSE and delta ----
#pragma unroll
            for (int i = 0; i < IPT; ++i) {
                const int it = tid + i * NT;
                if (it < ITEMS) {
                    const int rq = it / DCH;
                    const int dc = it - rq * DCH;
                    u32x4 qv[4], dvv[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int row = qb + 4 * rq + e;
                        if (row < sq && dc * 8 < p.head_dim) {
                            qv[e] = *reinterpret_cast<const u32x4*>(qbase + row * p.q_s + dc * 8);
                            dvv[e] = *reinterpret_cast<const u32x4*>(dobase + row * p.do_s + dc * 8);
                        } else {
                            qv[e] = u32x4{0, 0, 0, 0};
                            dvv[e] = u32x4{0, 0, 0, 0};
                        }
                        *reinterpret_cast<u32x4*>(&q_lds[(4 * rq + e) * RSTR + dc * 8]) = qv[e];
                        *reinterpret_cast<u32x4*>(&do_lds[(4 * rq + e) * RSTR + dc * 8]) = dvv[e];
                    }
#pragma unroll
                    for (int dd = 0; dd < 8; ++dd) {
                        const int w = dd >> 1, sh = (dd & 1) * 16;
                        uint2 a, c;
                        a.x = ((qv[0][w] >> sh) & 0xffffu) | (((qv[1][w] >> sh) & 0xffffu) << 16);
                        a.y = ((qv[2][w] >> sh) & 0xffffu) | (((qv[3][w] >> sh) & 0xffffu) << 16);
                        c.x = ((dvv[0][w] >> sh) & 0xffffu) | (((dvv[1][w] >> sh) & 0xffffu) << 16);
                        c.y = ((dvv[2][w] >> sh) & 0xffffu) | (((dvv[3][w] >> sh) & 0xffffu) << 16);
                        *reinterpret_cast<uint2*>(&qt_lds[(8 * dc + dd) * TSTR + 4 * rq]) = a;
                        *reinterpret_cast<uint2*>(&dot_lds[(8 * dc + dd) * TSTR + 4 * rq]) = c;
                    }
                }
            }
            for (int r = tid; r < BQ; r += NT) {
                const int row = qb + r;
                lse_lds[r] = row < sq ? lse_row[row] * kLog2e : INFINITY;
                dl_lds[r] = row < sq ? dl_row[row] : 0.0f;
            }
            __syncthreads();

            const bool need_mask = (key0 + BK > sk) || (wr >= 0 && key0 + BK - 1 > qb + off + wr) ||
                                   (wl >= 0 && key0 < qb + BQ - 1 + off - wl);

            u32x4 pP[4], pS[4];  // B operands, one per 16 queries of the tile
#pragma unroll
            for (int qc = 0; qc < 2; ++qc) {
                f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const u32x4 qa = *reinterpret_cast<const u32x4*>(&q_lds[(32 * qc + l32) * RSTR + 16 * ks + 8 * hh]);
                    const u32x4 da = *reinterpret_cast<const u32x4*>(&do_lds[(32 * qc + l32) * RSTR + 16 * ks + 8 * hh]);
                    s = mfma32<T>(qa, kf[ks], s);
                    dp = mfma32<T>(da, vf[ks], dp);
                }
                float pv[16], dsv[16];
                const uint32_t keep_bits =
                    p.drop_threshold < 255
                        ? keep_bits_key_lane(drop, static_cast<uint32_t>(b * p.heads + head),
                                             static_cast<uint32_t>(qb + 32 * qc), static_cast<uint32_t>(my_key), hh)
                        : 0xFFFFu;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int qloc = 32 * qc + 8 * g + 4 * hh;
                    const float4 lse4 = *reinterpret_cast<const float4*>(&lse_lds[qloc]);
                    const float4 dl4 = *reinterpret_cast<const float4*>(&dl_lds[qloc]);
                    const float lsev[4] = {lse4.x, lse4.y, lse4.z, lse4.w};
                    const float dlv[4] = {dl4.x, dl4.y, dl4.z, dl4.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int r = 4 * g + e;
                        const int row = qb + qloc + e;
                        float dfac;
                        const float x = bwd_score<GENERAL>(p, s[r], row, my_key, off, slope_log2, dfac);
                        float pr = fast_exp2(x - lsev[e]);
                        if (need_mask && masked_at(row, my_key, sk, off, wl, wr)) pr = 0.0f;
                        const bool kept = ((keep_bits >> r) & 1u) != 0u;
                        pv[r] = kept ? pr : 0.0f;
                        dsv[r] = pr * ((kept ? dp[r] : 0.0f) - dlv[e]) * dfac;
                    }
                }
#pragma unroll
                for (int t = 0; t < 2; ++t) {
#pragma unroll
                    for (int w = 0; w < 4; ++w) {
                        pP[2 * qc + t][w] = pack2<T>(pv[8 * t + 2 * w], pv[8 * t + 2 * w + 1]);
                        pS[2 * qc + t][w] = pack2<T>(dsv[8 * t + 2 * w], dsv[8 * t + 2 * w + 1]);
                    }
                }
            }

            // ---- dV^T += dO^T P, dK^T += Q^T dS ----
#pragma unroll
            for (int db = 0; db < DB; ++db) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int base = (32 * db + l32) * TSTR + 16 * t + 4 * hh;
                    const uint2 dlo = *reinterpret_cast<const uint2*>(&dot_lds[base]);
                    const uint2 dhi = *reinterpret_cast<const uint2*>(&dot_lds[base + 8]);
                    const uint2 qlo = *reinterpret_cast<const uint2*>(&qt_lds[base]);
                    const uint2 qhi = *reinterpret_cast<const uint2*>(&qt_lds[base + 8]);
                    dv[db] = mfma32<T>(u32x4{dlo.x, dlo.y, dhi.x, dhi.y}, pP[t], dv[db]);
                    dk[db] = mfma32<T>(u32x4{qlo.x, qlo.y, qhi.x, qhi.y}, pS[t], dk[db]);
                }
            }
            __syncthreads();
        }
    }

    // ---- write dK (times the softmax scale) and dV: lane = key, 4 consecutive d ----
    if (my_key < sk) {
        uint16_t* dkrow = static_cast<uint16_t*>(p.dk) + (VARLEN ? sb.k_off * p.dk_s : b * p.dk_b) +
                          kvh * p.dk_h + my_key * p.dk_s;
        uint16_t* dvrow = static_cast<uint16_t*>(p.dv) + (VARLEN ? sb.k_off * p.dv_s : b * p.dv_b) +
                          kvh * p.dv_h + my_key * p.dv_s;
        const float gs = p.grad_scale;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = 32 * db + 8 * g + 4 * hh;
                if (d < p.head_dim) {
                    uint2 a, c;
                    a.x = pack2<T>(dk[db][4 * g] * gs, dk[db][4 * g + 1] * gs);
                    a.y = pack2<T>(dk[db][4 * g + 2] * gs, dk[db][4 * g + 3] * gs);
                    c.x = pack2<T>(dv[db][4 * g] * p.inv_keep, dv[db][4 * g + 1] * p.inv_keep);
                    c.y = pack2<T>(dv[db][4 * g + 2] * p.inv_keep, dv[db][4 * g + 3] * p.inv_keep);
                    *reinterpret_cast<uint2*>(dkrow + d) = a;
                    *reinterpret_cast<uint2*>(dvrow + d) = c;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// dQ kernel.
// ---------------------------------------------------------------------------
template <typename T, int D, int NW, bool VARLEN, bool GENERAL>
__global__ void __launch_bounds__(NW * 64) flash_bwd_dq_kernel(const BwdParams p) {
    constexpr int BN = 64;
    constexpr int BM = 32 * NW;
    constexpr int NT = NW * 64;
    constexpr int KS = D / 16;
    constexpr int DB = D / 32;
    constexpr int RSTR = D + 8;
    constexpr int TSTR = BN + 8;
    constexpr int DCH = D / 8;
    constexpr int ITEMS = (BN / 4) * DCH;
    constexpr int IPT = (ITEMS + NT - 1) / NT;

    __shared__ __attribute__((aligned(16))) uint16_t k_lds[BN * RSTR];
    __shared__ __attribute__((aligned(16))) uint16_t v_lds[BN * RSTR];
    __shared__ __attribute__((aligned(16))) uint16_t kt_lds[D * TSTR];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, hh = lane >> 5;

    const int per = p.blocks_per_seq;
    const int qo = blockIdx.x % per;
    const int bh = blockIdx.x / per;
    const int b = bh / p.heads;
    const int head = bh - b * p.heads;
    const int kvh = head / p.gqa;
    const int qbi = per - 1 - qo;  // longest causal tiles first
    const SeqBounds sb = seq_bounds<VARLEN>(p, b);
    const DropoutState drop = p.drop_threshold < 255 ? dropout_state(p) : DropoutState{};
    if (!sb.ok) return;
    const int sq = sb.sq, sk = sb.sk;
    const int row0 = qbi * BM;
    if (row0 >= sq) return;
    const int off = sk - sq;
    const int wl = p.window_left, wr = p.window_right;

    const uint16_t* qbase = static_cast<const uint16_t*>(p.q) + (VARLEN ? sb.q_off * p.q_s : b * p.q_b) + head * p.q_h;
    const uint16_t* dobase = static_cast<const uint16_t*>(p.dout) + (VARLEN ? sb.q_off * p.do_s : b * p.do_b) + head * p.do_h;
    const uint16_t* kbase = static_cast<const uint16_t*>(p.k) + (VARLEN ? sb.k_off * p.k_s : b * p.k_b) + kvh * p.k_h;
    const uint16_t* vbase = static_cast<const uint16_t*>(p.v) + (VARLEN ? sb.k_off * p.v_s : b * p.v_b) + kvh * p.v_h;

    const int my_row = row0 + 32 * wave + l32;
    u32x4 qf[KS], dof[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const int d0 = 16 * ks + 8 * hh;
        if (my_row < sq && d0 < p.head_dim) {
            qf[ks] = *reinterpret_cast<const u32x4*>(qbase + my_row * p.q_s + d0);
            dof[ks] = *reinterpret_cast<const u32x4*>(dobase + my_row * p.do_s + d0);
        } else {
            qf[ks] = u32x4{0, 0, 0, 0};
            dof[ks] = u32x4{0, 0, 0, 0};
        }
    }
    float lse2 = INFINITY, dlt = 0.0f;
    if (my_row < sq) {
        lse2 = p.lse[(VARLEN ? 0 : b * p.lse_b) + head * p.lse_h + sb.lse_row0 + my_row] * kLog2e;
        dlt = p.delta[(VARLEN ? 0 : b * p.delta_b) + head * p.delta_h + sb.delta_row0 + my_row];
    }
    float slope_log2 = 0.0f;
    if constexpr (GENERAL) {
        if (p.alibi) slope_log2 = p.alibi[b * p.alibi_b + head] * kLog2e;
    }

    f32x16 acc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[db] = f32x16{};

    const int last_row = min(row0 + BM, sq) - 1;
    int kv_end = sk;
    if (wr >= 0) kv_end = max(0, min(sk, last_row + 1 + off + wr));
    int kv_begin = 0;
    if (wl >= 0) kv_begin = (max(0, min(sk, row0 + off - wl)) / BN) * BN;

    for (int kb = kv_begin; kb < kv_end; kb += BN) {
#pragma unroll
        for (int i = 0; i < IPT; ++i) {
            const int it = tid + i * NT;
            if (it < ITEMS) {
                const int kq = it / DCH;
                const int dc = it - kq * DCH;
                u32x4 kv4[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int key = kb + 4 * kq + e;
                    u32x4 vv = u32x4{0, 0, 0, 0};
                    kv4[e] = u32x4{0, 0, 0, 0};
                    if (key < sk && dc * 8 < p.head_dim) {
                        kv4[e] = *reinterpret_cast<const u32x4*>(kbase + key * p.k_s + dc * 8);
                        vv = *reinterpret_cast<const u32x4*>(vbase + key * p.v_s + dc * 8);
                    }
                    *reinterpret_cast<u32x4*>(&k_lds[(4 * kq + e) * RSTR + dc * 8]) = kv4[e];
                    *reinterpret_cast<u32x4*>(&v_lds[(4 * kq + e) * RSTR + dc * 8]) = vv;
                }
#pragma unroll
                for (int dd = 0; dd < 8; ++dd) {
                    const int w = dd >> 1, sh = (dd & 1) * 16;
                    uint2 a;
                    a.x = ((kv4[0][w] >> sh) & 0xffffu) | (((kv4[1][w] >> sh) & 0xffffu) << 16);
                    a.y = ((kv4[2][w] >> sh) & 0xffffu) | (((kv4[3][w] >> sh) & 0xffffu) << 16);
                    *reinterpret_cast<uint2*>(&kt_lds[(8 * dc + dd) * TSTR + 4 * kq]) = a;
                }
            }
        }
        __syncthreads();

        const bool need_mask = (kb + BN > sk) || (wr >= 0 && kb + BN - 1 > row0 + off + wr) ||
                               (wl >= 0 && kb < last_row + off - wl);
        // S^T and dP^T: lane = query, keys in registers.
        f32x16 s[2], dp[2];
        s[0] = s[1] = dp[0] = dp[1] = f32x16{};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
            for (int sub = 0; sub < 2; ++sub) {
                const u32x4 ka = *reinterpret_cast<const u32x4*>(&k_lds[(32 * sub + l32) * RSTR + 16 * ks + 8 * hh]);
                const u32x4 va = *reinterpret_cast<const u32x4*>(&v_lds[(32 * sub + l32) * RSTR + 16 * ks + 8 * hh]);
                s[sub] = mfma32<T>(ka, qf[ks], s[sub]);
                dp[sub] = mfma32<T>(va, dof[ks], dp[sub]);
            }
        }
        u32x4 pk[4];
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
            float dsv[16];
            const uint32_t keep_bits =
                p.drop_threshold < 255
                    ? keep_bits_query_lane(drop, static_cast<uint32_t>(b * p.heads + head),
                                           static_cast<uint32_t>(my_row), static_cast<uint32_t>(kb / 32 + sub), hh)
                    : 0xFFFFu;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int col = kb + 32 * sub + 8 * (r >> 2) + 4 * hh + (r & 3);
                float dfac;
                const float x = bwd_score<GENERAL>(p, s[sub][r], my_row, col, off, slope_log2, dfac);
                float pr = fast_exp2(x - lse2);
                if (need_mask && masked_at(my_row, col, sk, off, wl, wr)) pr = 0.0f;
                const bool kept = ((keep_bits >> r) & 1u) != 0u;
                dsv[r] = pr * ((kept ? dp[sub][r] : 0.0f) - dlt) * dfac;
            }
#pragma unroll
            for (int t = 0; t < 2; ++t) {
#pragma unroll
                for (int w = 0; w < 4; ++w) pk[2 * sub + t][w] = pack2<T>(dsv[8 * t + 2 * w], dsv[8 * t + 2 * w + 1]);
            }
        }
        // dQ^T += K^T dS^T
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int base = (32 * db + l32) * TSTR + 16 * t + 4 * hh;
                const uint2 lo = *reinterpret_cast<const uint2*>(&kt_lds[base]);
                const uint2 hi = *reinterpret_cast<const uint2*>(&kt_lds[base + 8]);
                acc[db] = mfma32<T>(u32x4{lo.x, lo.y, hi.x, hi.y}, pk[t], acc[db]);
            }
        }
        __syncthreads();
    }

    if (my_row < sq) {
        uint16_t* dqrow = static_cast<uint16_t*>(p.dq) + (VARLEN ? sb.q_off * p.dq_s : b * p.dq_b) +
                          head * p.dq_h + my_row * p.dq_s;
        const float gs = p.grad_scale;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = 32 * db + 8 * g + 4 * hh;
                if (d < p.head_dim) {
                    uint2 a;
                    a.x = pack2<T>(acc[db][4 * g] * gs, acc[db][4 * g + 1] * gs);
                    a.y = pack2<T>(acc[db][4 * g + 2] * gs, acc[db][4 * g + 3] * gs);
                    *reinterpret_cast<uint2*>(dqrow + d) = a;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Backward v2 (head size 64, 128 or 256; plain, dropout, softcap / ALiBi). Tiles are copied
// HBM -> LDS by direct buffer loads into row-major tiles whose 16-byte chunks are
// XOR-swizzled per row (kv_swizzle); the row-major reads are ds_read_b128 and
// every transposed MFMA operand (K^T in dQ, Q^T and dO^T in dK/dV) is read with
// ds_read_b64_tr_b16 from the same tile, so no transposed copy is ever stored.
// Two LDS stages, one barrier per tile; 2 waves per SIMD (D = 256: one block of
// 4 waves per CU, 128 KB of tiles and 512 registers per lane).
// ---------------------------------------------------------------------------

constexpr int kLook = 3;  // operand reads in flight ahead of their MFMA (v2 kernels)

template <typename T, int D, int NW, bool VARLEN, bool DROPOUT, int SCORED = 0>
__global__ void __launch_bounds__(NW * 64, D > 128 ? 1 : 8 / NW) flash_bwd_dq_v2_kernel(const BwdParams p) {
    constexpr int BN = 64;
    constexpr int BM = 32 * NW;
    constexpr int KS = D / 16;
    constexpr int DB = D / 32;
    constexpr int TILE = BN * D;

    __shared__ __attribute__((aligned(1024))) uint16_t k_lds[2 * TILE];
    __shared__ __attribute__((aligned(1024))) uint16_t v_lds[2 * TILE];

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar copy addresses
    const int l32 = lane & 31, hh = lane >> 5;
    TileLane<D> tl(lane);

    // Tile-major order, longest causal tiles first across the whole grid; the
    // query heads of one KV head share blockIdx % (B * Hk), hence one XCD when
    // B * Hk is a multiple of 8 (K/V tiles stay in that XCD's L2).
    const int per = p.blocks_per_seq;
    int b, kvh, head, qo;
    if (p.seq_major) {
        // Sequence-major: the blocks of one sequence run together and share its
        // K/V tiles in L2; the query heads of one KV head keep one XCD.
        const int nh = p.heads;
        b = blockIdx.x / (per * nh);
        const int rem = blockIdx.x - b * per * nh;
        qo = rem / nh;
        const int idx = rem - qo * nh;
        kvh = idx % p.kv_heads;
        head = kvh * p.gqa + idx / p.kv_heads;
    } else {
        const int nbh = p.batch * p.heads;
        const int nbkv = p.batch * p.kv_heads;
        qo = blockIdx.x / nbh;
        const int idx = blockIdx.x - qo * nbh;
        const int g = idx % nbkv;
        b = g / p.kv_heads;
        kvh = g - b * p.kv_heads;
        head = kvh * p.gqa + idx / nbkv;
    }
    const SeqBounds sb = seq_bounds<VARLEN>(p, b);
    DropoutState drop{};
    if constexpr (DROPOUT) drop = dropout_state(p);
    const uint32_t bh = static_cast<uint32_t>(b * p.heads + head);
    if (!sb.ok) return;
    const int sq = sb.sq, sk = sb.sk;
    // Counted from the end of this sequence (varlen sequences end at different tiles).
    const int qbi = (VARLEN ? (sq + BM - 1) / BM : per) - 1 - qo;
    if (qbi < 0) return;
    const int row0 = qbi * BM;
    if (row0 >= sq) return;
    const int off = sk - sq;
    const int wl = p.window_left, wr = p.window_right;

    const uint16_t* qbase = static_cast<const uint16_t*>(p.q) + (VARLEN ? sb.q_off * p.q_s : b * p.q_b) + head * p.q_h;
    const uint16_t* dobase = static_cast<const uint16_t*>(p.dout) + (VARLEN ? sb.q_off * p.do_s : b * p.do_b) + head * p.do_h;
    const uint16_t* kbase = static_cast<const uint16_t*>(p.k) + (VARLEN ? sb.k_off * p.k_s : b * p.k_b) + kvh * p.k_h;
    const uint16_t* vbase = static_cast<const uint16_t*>(p.v) + (VARLEN ? sb.k_off * p.v_s : b * p.v_b) + kvh * p.v_h;

    const int my_row = row0 + 32 * wave + l32;
    u32x4 qf[KS], dof[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const int d0 = 16 * ks + 8 * hh;
        const bool ok = my_row < sq;
        qf[ks] = ok ? *reinterpret_cast<const u32x4*>(qbase + my_row * p.q_s + d0) : u32x4{0, 0, 0, 0};
        dof[ks] = ok ? *reinterpret_cast<const u32x4*>(dobase + my_row * p.do_s + d0) : u32x4{0, 0, 0, 0};
    }
    float lse2 = INFINITY, dlt = 0.0f;
    if (my_row < sq) {
        lse2 = p.lse[(VARLEN ? 0 : b * p.lse_b) + head * p.lse_h + sb.lse_row0 + my_row] * kLog2e;
        dlt = p.delta[(VARLEN ? 0 : b * p.delta_b) + head * p.delta_h + sb.delta_row0 + my_row];
    }
    const float c = p.scale_log2;
    [[maybe_unused]] float slope_log2 = 0.0f;
    if constexpr (SCORED) {
        if (p.alibi) slope_log2 = p.alibi[b * p.alibi_b + head] * kLog2e;
    }

    f32x16 acc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[db] = f32x16{};

    const int last_row = min(row0 + BM, sq) - 1;
    int kv_end = sk;
    if (wr >= 0) kv_end = max(0, min(sk, last_row + 1 + off + wr));
    int kv_begin = 0;
    if (wl >= 0) kv_begin = (max(0, min(sk, row0 + off - wl)) / BN) * BN;
    const int ntiles = kv_begin < kv_end ? (kv_end - kv_begin + BN - 1) / BN : 0;

    auto copy_tile = [&](int kb, int stage) {
        copy_rows_dma<D, NW, 64>(kbase + static_cast<int64_t>(kb) * p.k_s, p.k_s, sk - kb, k_lds + stage * TILE, wave, lane);
        copy_rows_dma<D, NW, 64>(vbase + static_cast<int64_t>(kb) * p.v_s, p.v_s, sk - kb, v_lds + stage * TILE, wave, lane);
    };
    if (ntiles > 0) {
        copy_tile(kv_begin, 0);
        wait_vmem();
        __syncthreads();
    }

    for (int t = 0; t < ntiles; ++t) {
        const int kb = kv_begin + t * BN;
        tl.refresh();
        const uint16_t* kl = k_lds + (t & 1) * TILE;
        const uint16_t* vl = v_lds + (t & 1) * TILE;
        if (t + 1 < ntiles) copy_tile(kb + BN, (t + 1) & 1);

        // S^T = K Q^T and dP^T = V dO^T: step i reads K (even i) or V (odd i) of
        // key half (i / 2) % 2 at k-step i / 4, kLook MFMAs ahead of its use.
        f32x16 s[2], dp[2];
        s[0] = s[1] = dp[0] = dp[1] = f32x16{};
        {
            constexpr int N = 4 * KS;
            auto load = [&](auto ic) __attribute__((always_inline)) -> u32x4 {
                constexpr int i = decltype(ic)::value;
                return tl.rm((i & 1) ? vl : kl, (i >> 1) & 1, i >> 2);
            };
            u32x4 ring[kLook];
            static_for<0, kLook>([&](auto ic) __attribute__((always_inline)) { ring[decltype(ic)::value] = load(ic); });
            __builtin_amdgcn_sched_group_barrier(0x100, kLook, 0);
            static_for<0, N>([&](auto ic) __attribute__((always_inline)) {
                constexpr int i = decltype(ic)::value;
                constexpr int sub = (i >> 1) & 1, ks = i >> 2;
                const u32x4 a = ring[i % kLook];
                if constexpr (i + kLook < N) {
                    ring[i % kLook] = load(std::integral_constant<int, i + kLook>{});
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                if constexpr (i & 1) {
                    dp[sub] = mfma32<T>(a, dof[ks], dp[sub]);
                } else {
                    s[sub] = mfma32<T>(a, qf[ks], s[sub]);
                }
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            });
        }
        const bool need_mask = (kb + BN > sk) || (wr >= 0 && kb + BN - 1 > row0 + off + wr) ||
                               (wl >= 0 && kb < last_row + off - wl);
        u32x4 pk[4];
        // The mask test is hoisted out of the element loop: one branch per
        // tile instead of a scalar branch per element.
        // MASK: 0 none, 1 masked, 2 tested per element (the dropout and scored
        // kernels, where two copies of the loop would spill).
        auto ds_tile = [&](auto mask_tag) __attribute__((always_inline)) {
            constexpr int MASK = decltype(mask_tag)::value;
#pragma unroll
            for (int sub = 0; sub < 2; ++sub) {
                float dsv[16];
                // Dropped entries of dP are zeroed (dS = P (dP M - delta)).
                if constexpr (DROPOUT) {
                    apply_dropout_query_lane(drop, bh, static_cast<uint32_t>(my_row),
                                             static_cast<uint32_t>(kb / 32 + sub), hh, dp[sub]);
                }
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int col = kb + 32 * sub + 8 * (r >> 2) + 4 * hh + (r & 3);
                    float dfac;
                    float pr = bwd_prob<SCORED>(p, s[sub][r], c, lse2, my_row, col, off, slope_log2, dfac);
                    if (MASK == 1 || (MASK == 2 && need_mask)) {
                        const bool masked = (col >= sk) | (wr >= 0 & col > my_row + off + wr) |
                                            (wl >= 0 & col < my_row + off - wl);
                        pr = masked ? 0.0f : pr;
                    }
                    dsv[r] = pr * (dp[sub][r] - dlt) * dfac;
                }
#pragma unroll
                for (int t2 = 0; t2 < 2; ++t2) {
#pragma unroll
                    for (int w = 0; w < 4; ++w) {
                        pk[2 * sub + t2][w] = pack2<T>(dsv[8 * t2 + 2 * w], dsv[8 * t2 + 2 * w + 1]);
                    }
                }
            }
        };
        if constexpr (DROPOUT || SCORED != 0) {
            ds_tile(std::integral_constant<int, 2>{});
        } else if (need_mask) {
            ds_tile(std::integral_constant<int, 1>{});
        } else {
            ds_tile(std::integral_constant<int, 0>{});
        }
        // dQ^T += K^T dS^T (K^T read transposed from the key tile); step i:
        // db = i % DB, tt = i / DB, reads ahead as above.
        {
            constexpr int N = 4 * DB;
            u32x4 ring[kLook];
            static_for<0, kLook>([&](auto ic) __attribute__((always_inline)) {
                constexpr int i = decltype(ic)::value;
                ring[i] = tl.tr(kl, i % DB, i / DB);
            });
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * kLook, 0);
            static_for<0, N>([&](auto ic) __attribute__((always_inline)) {
                constexpr int i = decltype(ic)::value;
                const u32x4 a = ring[i % kLook];
                if constexpr (i + kLook < N) {
                    ring[i % kLook] = tl.tr(kl, (i + kLook) % DB, (i + kLook) / DB);
                    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                }
                acc[i % DB] = mfma32<T>(a, pk[i / DB], acc[i % DB]);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            });
        }
        wait_vmem();
        __syncthreads();
    }

    if (my_row < sq) {
        uint16_t* dqrow = static_cast<uint16_t*>(p.dq) + (VARLEN ? sb.q_off * p.dq_s : b * p.dq_b) +
                          head * p.dq_h + my_row * p.dq_s;
        const float gs = p.grad_scale;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = 32 * db + 8 * g + 4 * hh;
                uint2 a;
                a.x = pack2<T>(acc[db][4 * g] * gs, acc[db][4 * g + 1] * gs);
                a.y = pack2<T>(acc[db][4 * g + 2] * gs, acc[db][4 * g + 3] * gs);
                *reinterpret_cast<uint2*>(dqrow + d) = a;
            }
        }
    }
}

template <typename T, int D, int NW, bool VARLEN, bool DROPOUT, bool PAIRED, int SCORED = 0>
__global__ void __launch_bounds__(NW * 64, D > 128 ? 1 : 8 / NW) flash_bwd_dkv_v2_kernel(const BwdParams p) {
    // D = 128: the dK and dV accumulators (128 registers) and K (32) leave no
    // room for V in registers at 2 waves per SIMD, so V is staged once in LDS
    // and the query tiles shrink to 32 rows to keep two blocks per CU.
    constexpr bool V_LDS = D > 64;
    constexpr int BK = 32 * NW;
    constexpr int BQ = V_LDS ? 32 : 64;
    constexpr int NQC = BQ / 32;
    constexpr int KS = D / 16;
    constexpr int DB = D / 32;
    constexpr int TILE = BQ * D;
    static_assert(NW >= 2, "two waves stage the LSE and delta rows");

    __shared__ __attribute__((aligned(1024))) uint16_t q_lds[2 * TILE];
    __shared__ __attribute__((aligned(1024))) uint16_t do_lds[2 * TILE];
    __shared__ __attribute__((aligned(1024))) uint16_t v_lds[V_LDS ? BK * D : 8];
    // 64 entries per stage: a 4-byte direct copy always writes a whole wave.
    __shared__ __attribute__((aligned(16))) float lse_lds[2 * 64];
    __shared__ __attribute__((aligned(16))) float dl_lds[2 * 64];

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar copy addresses
    const int l32 = lane & 31, hh = lane >> 5;
    TileLane<D> tl(lane);

    // Tile-major order: the key tiles that see the most causal queries start
    // first across the whole grid; one (batch, KV head) keeps one XCD.
    int b, kvh, kbi;
    int kbi2 = -1;  // the second key tile of a paired block
    if constexpr (PAIRED) {
        // Masked dense grids: block pr of a (batch, KV head) group takes key
        // tiles pr and per - 1 - pr, whose causal work adds up to the same for
        // every block. With equal blocks the grid runs group-major per XCD
        // (blocks go to XCD blockIdx % 8): one group's Q / dO tiles are read by
        // the blocks of one XCD at a time.
        const int per = p.blocks_per_seq;
        const int npairs = (per + 1) / 2;
        int g, pr;
        if ((p.batch * p.kv_heads) % 8 == 0) {
            const int xcd = static_cast<int>(blockIdx.x) & 7;
            const int k = static_cast<int>(blockIdx.x) >> 3;
            const int gl = k / npairs;
            pr = k - gl * npairs;
            g = gl * 8 + xcd;
        } else {
            g = static_cast<int>(blockIdx.x) / npairs;
            pr = static_cast<int>(blockIdx.x) - g * npairs;
        }
        b = g / p.kv_heads;
        kvh = g - b * p.kv_heads;
        kbi = pr;
        kbi2 = per - 1 - pr;
        if (kbi2 == kbi) kbi2 = -1;
    } else if (p.seq_major) {
        // Sequence-major (see the dQ kernel): key tiles of one sequence together.
        const int per = p.blocks_per_seq;
        b = blockIdx.x / (per * p.kv_heads);
        const int rem = blockIdx.x - b * per * p.kv_heads;
        kbi = rem / p.kv_heads;
        kvh = rem - kbi * p.kv_heads;
    } else {
        const int nbkv = p.batch * p.kv_heads;
        kbi = blockIdx.x / nbkv;
        const int bkv = blockIdx.x - kbi * nbkv;
        b = bkv / p.kv_heads;
        kvh = bkv - b * p.kv_heads;
    }
    const SeqBounds sb = seq_bounds<VARLEN>(p, b);
    DropoutState drop{};
    if constexpr (DROPOUT) drop = dropout_state(p);
    if (!sb.ok) return;
    const int sq = sb.sq, sk = sb.sk;
    // One key tile, or two for a paired block (the body is inlined once per
    // tile, so the two copies' registers do not overlap); the tile loop's last
    // barrier orders the second tile's V and Q / dO staging after every read
    // of the first.
    auto key_tile = [&](const int kt) __attribute__((always_inline)) {
        const int key0 = kt * BK;
        if (key0 >= sk) return;
        const int off = sk - sq;
        const int wl = p.window_left, wr = p.window_right;

        const uint16_t* kbase = static_cast<const uint16_t*>(p.k) + (VARLEN ? sb.k_off * p.k_s : b * p.k_b) + kvh * p.k_h;
        const uint16_t* vbase = static_cast<const uint16_t*>(p.v) + (VARLEN ? sb.k_off * p.v_s : b * p.v_b) + kvh * p.v_h;

        // This wave's 32 keys: K (and V) rows as B operands of S = Q K^T, dP = dO V^T.
        const int my_key = key0 + 32 * wave + l32;
        u32x4 kf[KS];
        u32x4 vf[V_LDS ? 1 : KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int d0 = 16 * ks + 8 * hh;
            const bool ok = my_key < sk;
            kf[ks] = ok ? *reinterpret_cast<const u32x4*>(kbase + my_key * p.k_s + d0) : u32x4{0, 0, 0, 0};
            if constexpr (!V_LDS) {
                vf[ks] = ok ? *reinterpret_cast<const u32x4*>(vbase + my_key * p.v_s + d0) : u32x4{0, 0, 0, 0};
            }
        }
        if constexpr (V_LDS) {
            copy_rows_dma<D, NW, BK>(vbase + static_cast<int64_t>(key0) * p.v_s, p.v_s, sk - key0, v_lds, wave, lane);
        }
        f32x16 dk[DB], dv[DB];
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            dk[db] = f32x16{};
            dv[db] = f32x16{};
        }

        // Query rows that can see some key of this block.
        const int key_last = min(key0 + BK, sk) - 1;
        int q_begin = 0;
        if (wr >= 0) q_begin = max(0, key0 - off - wr);
        q_begin = (q_begin / BQ) * BQ;
        int q_end = sq;
        if (wl >= 0) q_end = max(0, min(sq, key_last - off + wl + 1));
        const int nqb = q_begin < q_end ? (q_end - q_begin + BQ - 1) / BQ : 0;
        // (query tile, query head of the group) pairs, last query tile first: the
        // key blocks of one (batch, KV head) run on one XCD and all end at the last
        // query tile, so walking the tiles downward keeps them reading the same
        // Q / dO tiles at the same time (shared through L2).
        const int gqa = p.gqa;
        const int ntiles = nqb * gqa;
        const float c = p.scale_log2;
        [[maybe_unused]] float slope_log2 = 0.0f;  // per query head (tj), set per tile

        // Tile t is query tile nqb - 1 - t / gqa (counted from q_begin) of query
        // head kvh * gqa + t % gqa. The copies walk that order with a cursor of row
        // pointers stepped per tile (no division or 64-bit multiply per tile).
        struct Cursor {
            int j, qb;  // head within the group, first query row of the tile
            const uint16_t* q;
            const uint16_t* dout;
            const float* lse;
            const float* delta;
        };
        const int qb_last = q_begin + (nqb - 1) * BQ;
        Cursor cur;
        {
            const int head0 = kvh * gqa;
            cur.j = 0;
            cur.qb = qb_last;
            cur.q = static_cast<const uint16_t*>(p.q) + (VARLEN ? sb.q_off * p.q_s : b * p.q_b) + head0 * p.q_h +
                    static_cast<int64_t>(qb_last) * p.q_s;
            cur.dout = static_cast<const uint16_t*>(p.dout) + (VARLEN ? sb.q_off * p.do_s : b * p.do_b) +
                       head0 * p.do_h + static_cast<int64_t>(qb_last) * p.do_s;
            cur.lse = p.lse + (VARLEN ? 0 : b * p.lse_b) + head0 * p.lse_h + sb.lse_row0 + qb_last;
            cur.delta = p.delta + (VARLEN ? 0 : b * p.delta_b) + head0 * p.delta_h + sb.delta_row0 + qb_last;
        }
        // Steps when the head index wraps: back to the group's first head, one
        // query tile down.
        const int64_t q_wrap = -static_cast<int64_t>(gqa) * p.q_h - static_cast<int64_t>(BQ) * p.q_s;
        const int64_t do_wrap = -static_cast<int64_t>(gqa) * p.do_h - static_cast<int64_t>(BQ) * p.do_s;
        const int64_t lse_wrap = -static_cast<int64_t>(gqa) * p.lse_h - BQ;
        const int64_t delta_wrap = -static_cast<int64_t>(gqa) * p.delta_h - BQ;
        auto advance = [&](Cursor& c) {
            ++c.j;
            c.q += p.q_h;
            c.dout += p.do_h;
            c.lse += p.lse_h;
            c.delta += p.delta_h;
            if (c.j == gqa) {
                c.j = 0;
                c.qb -= BQ;
                c.q += q_wrap;
                c.dout += do_wrap;
                c.lse += lse_wrap;
                c.delta += delta_wrap;
            }
        };
        auto copy_tile = [&](const Cursor& c, int stage) {
            copy_rows_dma<D, NW, BQ>(c.q, p.q_s, sq - c.qb, q_lds + stage * TILE, wave, lane);
            copy_rows_dma<D, NW, BQ>(c.dout, p.do_s, sq - c.qb, do_lds + stage * TILE, wave, lane);
            // Rows past the sequence read LSE 0 and delta 0; their Q and dO rows are
            // zero, so they add nothing to dK and dV.
            const uint32_t rows = static_cast<uint32_t>(max(0, min(sq - c.qb, BQ)));
            if (wave == 0) {
                dma_lds4(rsrc_words(c.lse, rows * 4u), lds_addr(lse_lds + stage * 64), lane * 4u);
            } else if (wave == 1) {
                dma_lds4(rsrc_words(c.delta, rows * 4u), lds_addr(dl_lds + stage * 64), lane * 4u);
            }
        };
        if (ntiles > 0) copy_tile(cur, 0);
        wait_vmem();
        __syncthreads();
        int tj = 0, qb = qb_last;  // the computed tile's head index and first row

        for (int t = 0; t < ntiles; ++t) {
            tl.refresh();
            const int stage = t & 1;
            const uint16_t* ql = q_lds + stage * TILE;
            const uint16_t* dl = do_lds + stage * TILE;
            const float* lsl = lse_lds + stage * 64;
            const float* dll = dl_lds + stage * 64;
            if (t + 1 < ntiles) {
                advance(cur);
                copy_tile(cur, stage ^ 1);
            }
            if constexpr (SCORED) {
                if (p.alibi) slope_log2 = p.alibi[b * p.alibi_b + kvh * gqa + tj] * kLog2e;
            }

            const bool need_mask = (key0 + BK > sk) || (wr >= 0 && key0 + BK - 1 > qb + off + wr) ||
                                   (wl >= 0 && key0 < qb + BQ - 1 + off - wl);
#pragma unroll
            for (int qc = 0; qc < NQC; ++qc) {
                // S = Q K^T and dP = dO V^T; the operands of k-step ks + 1 are read
                // while the MFMAs of k-step ks run.
                f32x16 s = f32x16{}, dp = f32x16{};
                {
                    constexpr int NR = V_LDS ? 3 : 2;
                    auto rd = [&](auto ic, u32x4 (&r)[NR]) __attribute__((always_inline)) {
                        constexpr int ks = decltype(ic)::value;
                        r[0] = tl.rm(ql, qc, ks);
                        r[1] = tl.rm(dl, qc, ks);
                        if constexpr (V_LDS) r[2] = tl.rm(v_lds, wave, ks);
                    };
                    u32x4 ra[2][NR];
                    rd(std::integral_constant<int, 0>{}, ra[0]);
                    __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
                    static_for<0, KS>([&](auto ic) __attribute__((always_inline)) {
                        constexpr int ks = decltype(ic)::value;
                        if constexpr (ks + 1 < KS) {
                            rd(std::integral_constant<int, ks + 1>{}, ra[(ks + 1) & 1]);
                            __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
                        }
                        const u32x4(&r)[NR] = ra[ks & 1];
                        s = mfma32<T>(r[0], kf[ks], s);
                        if constexpr (V_LDS) {
                            dp = mfma32<T>(r[1], r[2], dp);
                        } else {
                            dp = mfma32<T>(r[1], vf[ks], dp);
                        }
                        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                    });
                }
                u32x4 pP[2], pS[2];
                float pv[16], dsv[16];
                uint32_t keep_bits = 0xFFFFu;
                if constexpr (DROPOUT) {
                    keep_bits = keep_bits_key_lane_shared(drop, static_cast<uint32_t>(b * p.heads + kvh * gqa + tj),
                                                   static_cast<uint32_t>(qb + 32 * qc), static_cast<uint32_t>(my_key), hh);
                }
                // The mask test is hoisted out of the element loop: one branch per
                // tile instead of a scalar branch per element.
                auto p_ds = [&](auto mask_tag) __attribute__((always_inline)) {
                    constexpr bool MASK = decltype(mask_tag)::value;
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int qloc = 32 * qc + 8 * g + 4 * hh;
                        const float4 l4 = *reinterpret_cast<const float4*>(lsl + qloc);
                        const float4 d4 = *reinterpret_cast<const float4*>(dll + qloc);
                        const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
                        const float dv4[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int r = 4 * g + e;
                            const int prow = qb + qloc + e;
                            float dfac;
                            float pr = bwd_prob<SCORED>(p, s[r], c, lv[e] * kLog2e, prow, my_key, off, slope_log2, dfac);
                            // Rows past the sequence read LSE 0 and zero Q / dO rows: a
                            // plain score is 0 there, but an ALiBi bias alone can
                            // overflow P (then inf x 0 in the dV MFMA).
                            if constexpr (SCORED) pr = prow < sq ? pr : 0.0f;
                            if constexpr (MASK) {
                                const int row = qb + qloc + e;
                                const bool masked = (my_key >= sk) | (wr >= 0 & my_key > row + off + wr) |
                                                    (wl >= 0 & my_key < row + off - wl);
                                pr = masked ? 0.0f : pr;
                            }
                            const bool kept = ((keep_bits >> r) & 1u) != 0u;
                            pv[r] = kept ? pr : 0.0f;
                            dsv[r] = pr * ((kept ? dp[r] : 0.0f) - dv4[e]) * dfac;
                        }
                    }
                };
                if constexpr (DROPOUT || SCORED != 0) {
                    // The dropout and scored kernels keep the per-element test
                    // inline: two inlined copies of the loop spill.
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int qloc = 32 * qc + 8 * g + 4 * hh;
                        const float4 l4 = *reinterpret_cast<const float4*>(lsl + qloc);
                        const float4 d4 = *reinterpret_cast<const float4*>(dll + qloc);
                        const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
                        const float dv4[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int r = 4 * g + e;
                            const int prow = qb + qloc + e;
                            float dfac;
                            float pr = bwd_prob<SCORED>(p, s[r], c, lv[e] * kLog2e, prow, my_key, off, slope_log2, dfac);
                            // Rows past the sequence read LSE 0 and zero Q / dO rows: a
                            // plain score is 0 there, but an ALiBi bias alone can
                            // overflow P (then inf x 0 in the dV MFMA).
                            if constexpr (SCORED) pr = prow < sq ? pr : 0.0f;
                            if (need_mask) {
                                const int row = qb + qloc + e;
                                const bool masked = (my_key >= sk) | (wr >= 0 & my_key > row + off + wr) |
                                                    (wl >= 0 & my_key < row + off - wl);
                                pr = masked ? 0.0f : pr;
                            }
                            const bool kept = ((keep_bits >> r) & 1u) != 0u;
                            pv[r] = kept ? pr : 0.0f;
                            dsv[r] = pr * ((kept ? dp[r] : 0.0f) - dv4[e]) * dfac;
                        }
                    }
                } else if (need_mask) {
                    p_ds(std::true_type{});
                } else {
                    p_ds(std::false_type{});
                }
#pragma unroll
                for (int t2 = 0; t2 < 2; ++t2) {
#pragma unroll
                    for (int w = 0; w < 4; ++w) {
                        pP[t2][w] = pack2<T>(pv[8 * t2 + 2 * w], pv[8 * t2 + 2 * w + 1]);
                        pS[t2][w] = pack2<T>(dsv[8 * t2 + 2 * w], dsv[8 * t2 + 2 * w + 1]);
                    }
                }
                // dV^T += dO^T P and dK^T += Q^T dS (transposed reads of the query
                // tiles), step i = (db, t2) with the next step's operands in flight.
                {
                    auto rd = [&](auto ic, u32x4 (&r)[2]) __attribute__((always_inline)) {
                        constexpr int i = decltype(ic)::value;
                        r[0] = tl.tr(dl, i >> 1, 2 * qc + (i & 1));
                        r[1] = tl.tr(ql, i >> 1, 2 * qc + (i & 1));
                    };
                    u32x4 rb[2][2];
                    rd(std::integral_constant<int, 0>{}, rb[0]);
                    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
                    static_for<0, 2 * DB>([&](auto ic) __attribute__((always_inline)) {
                        constexpr int i = decltype(ic)::value;
                        constexpr int db = i >> 1, t2 = i & 1;
                        if constexpr (i + 1 < 2 * DB) {
                            rd(std::integral_constant<int, i + 1>{}, rb[(i + 1) & 1]);
                            __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
                        }
                        const u32x4(&r)[2] = rb[i & 1];
                        dv[db] = mfma32<T>(r[0], pP[t2], dv[db]);
                        dk[db] = mfma32<T>(r[1], pS[t2], dk[db]);
                        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                    });
                }
            }
            if (++tj == gqa) {
                tj = 0;
                qb -= BQ;
            }
            wait_vmem();
            __syncthreads();
        }

        if (my_key < sk) {
            uint16_t* dkrow = static_cast<uint16_t*>(p.dk) + (VARLEN ? sb.k_off * p.dk_s : b * p.dk_b) +
                              kvh * p.dk_h + my_key * p.dk_s;
            uint16_t* dvrow = static_cast<uint16_t*>(p.dv) + (VARLEN ? sb.k_off * p.dv_s : b * p.dv_b) +
                              kvh * p.dv_h + my_key * p.dv_s;
            const float gs = p.grad_scale;
#pragma unroll
            for (int db = 0; db < DB; ++db) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int d = 32 * db + 8 * g + 4 * hh;
                    uint2 a, cc;
                    a.x = pack2<T>(dk[db][4 * g] * gs, dk[db][4 * g + 1] * gs);
                    a.y = pack2<T>(dk[db][4 * g + 2] * gs, dk[db][4 * g + 3] * gs);
                    cc.x = pack2<T>(dv[db][4 * g] * p.inv_keep, dv[db][4 * g + 1] * p.inv_keep);
                    cc.y = pack2<T>(dv[db][4 * g + 2] * p.inv_keep, dv[db][4 * g + 3] * p.inv_keep);
                    *reinterpret_cast<uint2*>(dkrow + d) = a;
                    *reinterpret_cast<uint2*>(dvrow + d) = cc;
                }
            }
        }
    };
    key_tile(kbi);
    // Only the paired instance carries a second inlined copy of the body
    // (the dropout kernel's would not fit the registers of two waves per SIMD).
    if constexpr (PAIRED) {
        if (kbi2 >= 0) key_tile(kbi2);
    }
}

__global__ void zero_u16_kernel(uint16_t* x, int64_t n) {
    for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += gridDim.x * 256ll) x[i] = 0;
}

__global__ void zero_f32_kernel(float* x, int64_t n) {
    for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += gridDim.x * 256ll) x[i] = 0.0f;
}

}  // namespace attn

namespace {

using namespace attn;

constexpr int kDkvWaves = 4;
constexpr int kDqWaves = 4;

void zero_u16(void* x, int64_t n, hipStream_t s) {
    if (n <= 0) return;
    zero_u16_kernel<<<static_cast<unsigned>(std::min<int64_t>((n + 255) / 256, 65536)), 256, 0, s>>>(
        static_cast<uint16_t*>(x), n);
    check_launch("zero gradient");
}

void zero_f32(float* x, int64_t n, hipStream_t s) {
    if (n <= 0) return;
    zero_f32_kernel<<<static_cast<unsigned>(std::min<int64_t>((n + 255) / 256, 65536)), 256, 0, s>>>(x, n);
    check_launch("zero delta");
}

template <typename T, int D, bool VARLEN, int DKV_WAVES, int DQ_WAVES, bool DROPOUT, int SCORED>
void launch_bwd_v2(BwdParams prm, bool want_q, bool want_kv, hipStream_t s) {
    if (want_kv) {
        constexpr int BK = 32 * DKV_WAVES;
        prm.blocks_per_seq = (prm.seqlen_k + BK - 1) / BK;
        // Paired blocks take two key tiles each (see the kernel).
        const int64_t per_group = prm.pair_tiles ? (prm.blocks_per_seq + 1) / 2 : prm.blocks_per_seq;
        const int64_t blocks = per_group * prm.batch * prm.kv_heads;
        if (blocks > 0) {
            const unsigned grid = static_cast<unsigned>(blocks);
            if constexpr (!VARLEN && !DROPOUT && SCORED == 0 && D != 256) {
                if (prm.pair_tiles) {
                    flash_bwd_dkv_v2_kernel<T, D, DKV_WAVES, false, false, true><<<grid, DKV_WAVES * 64, 0, s>>>(prm);
                } else {
                    flash_bwd_dkv_v2_kernel<T, D, DKV_WAVES, false, false, false><<<grid, DKV_WAVES * 64, 0, s>>>(prm);
                }
            } else {
                flash_bwd_dkv_v2_kernel<T, D, DKV_WAVES, VARLEN, DROPOUT, false, SCORED>
                    <<<grid, DKV_WAVES * 64, 0, s>>>(prm);
            }
            check_launch("launch flash_bwd_dkv");
        }
    }
    if (want_q) {
        constexpr int BM = 32 * DQ_WAVES;
        prm.blocks_per_seq = (prm.seqlen_q + BM - 1) / BM;
        const int64_t blocks = static_cast<int64_t>(prm.blocks_per_seq) * prm.batch * prm.heads;
        if (blocks > 0) {
            flash_bwd_dq_v2_kernel<T, D, DQ_WAVES, VARLEN, DROPOUT, SCORED>
                <<<static_cast<unsigned>(blocks), DQ_WAVES * 64, 0, s>>>(prm);
            check_launch("launch flash_bwd_dq");
        }
    }
}

template <typename T, int D, bool VARLEN, bool GEN>
void launch_bwd_t(BwdParams prm, bool want_q, bool want_kv, hipStream_t s) {
    if constexpr (D == 64 || D == 128 || D == 256) {
        // The tiled kernels need the full bucket width and 32-bit tile offsets.
        constexpr int64_t kMaxStride = int64_t{1} << 23;
        auto ok = [&](int64_t st) { return st >= 0 && st <= kMaxStride; };
        const bool fits = prm.head_dim == D && ok(prm.q_s) && ok(prm.k_s) && ok(prm.v_s) && ok(prm.do_s);
        if (fits) {
            // Sequence-major block order when every block of a sequence does the
            // same work (no causal / window mask) or the sequences are packed:
            // concurrent blocks then share one sequence's tiles in L2. Masked
            // dense grids keep the tile-major, longest-first order.
            prm.seq_major = (VARLEN || (prm.window_left < 0 && prm.window_right < 0)) ? 1 : 0;
            // Softcap / ALiBi (GEN): the scored instances (1: ALiBi only, 2:
            // softcap with or without ALiBi), unpaired.
            // D = 256 (one block per CU) runs unpaired: 581 -> 614 TFLOP/s causal.
            prm.pair_tiles = (prm.seq_major || prm.drop_threshold < 255 || GEN || D == 256) ? 0 : 1;
            auto go = [&](auto mode_tag) {
                constexpr int MODE = decltype(mode_tag)::value;
                if (prm.drop_threshold < 255) {
                    launch_bwd_v2<T, D, VARLEN, 4, 4, true, MODE>(prm, want_q, want_kv, s);
                } else {
                    launch_bwd_v2<T, D, VARLEN, 4, 4, false, MODE>(prm, want_q, want_kv, s);
                }
            };
            if constexpr (GEN) {
                if (prm.tanh_scale > 0.0f) {
                    go(std::integral_constant<int, 2>{});
                } else {
                    go(std::integral_constant<int, 1>{});
                }
            } else {
                go(std::integral_constant<int, 0>{});
            }
            return;
        }
    }
    if (want_kv) {
        constexpr int BK = 32 * kDkvWaves;
        prm.blocks_per_seq = (prm.seqlen_k + BK - 1) / BK;
        const int64_t blocks = static_cast<int64_t>(prm.blocks_per_seq) * prm.batch * prm.kv_heads;
        if (blocks > 0) {
            flash_bwd_dkv_kernel<T, D, kDkvWaves, VARLEN, GEN><<<static_cast<unsigned>(blocks), kDkvWaves * 64, 0, s>>>(prm);
            check_launch("launch flash_bwd_dkv");
        }
    }
    if (want_q) {
        constexpr int BM = 32 * kDqWaves;
        prm.blocks_per_seq = (prm.seqlen_q + BM - 1) / BM;
        const int64_t blocks = static_cast<int64_t>(prm.blocks_per_seq) * prm.batch * prm.heads;
        if (blocks > 0) {
            flash_bwd_dq_kernel<T, D, kDqWaves, VARLEN, GEN><<<static_cast<unsigned>(blocks), kDqWaves * 64, 0, s>>>(prm);
            check_launch("launch flash_bwd_dq");
        }
    }
}

template <bool VARLEN>
void launch_bwd(const BwdParams& prm, int dtype, int bucket, bool general, bool want_q, bool want_kv,
                hipStream_t s) {
    auto with_t = [&](auto tag) {
        using T = decltype(tag);
        auto with_d = [&](auto dtag) {
            constexpr int D = decltype(dtag)::value;
            if (general) {
                launch_bwd_t<T, D, VARLEN, true>(prm, want_q, want_kv, s);
            } else {
                launch_bwd_t<T, D, VARLEN, false>(prm, want_q, want_kv, s);
            }
        };
        switch (bucket) {
            case 32: with_d(std::integral_constant<int, 32>{}); break;
            case 64: with_d(std::integral_constant<int, 64>{}); break;
            case 96: with_d(std::integral_constant<int, 96>{}); break;
            case 128: with_d(std::integral_constant<int, 128>{}); break;
            case 160: with_d(std::integral_constant<int, 160>{}); break;
            case 192: with_d(std::integral_constant<int, 192>{}); break;
            case 224: with_d(std::integral_constant<int, 224>{}); break;
            case 256: with_d(std::integral_constant<int, 256>{}); break;
            default: throw value_error("unsupported head dim bucket " + std::to_string(bucket));
        }
    };
    if (dtype == KCR_BFLOAT16) {
        with_t(bf16_t{});
    } else {
        with_t(f16_t{});
    }
}

void check_grad(const kcr_tensor* g, const kcr_tensor* like, const char* name) {
    if (!g) return;
    if (shape_of(*g) != shape_of(*like) || g->dtype != like->dtype) {
        throw value_error(std::string(name) + " must match its input's shape and dtype");
    }
    if (!rows_aligned16(g) || g->strides[g->ndim - 1] != 1) {
        throw value_error(std::string(name) + " must have unit last stride and 16-byte aligned rows");
    }
    require_device(g, name);
}

void check_f32_tensor(const kcr_tensor* t, const std::vector<int64_t>& shape, const char* name) {
    if (!t || t->dtype != KCR_FLOAT32 || shape_of(*t) != shape || !is_contiguous(*t)) {
        throw value_error(std::string(name) + " must be contiguous float32 with shape " + shape_string(shape));
    }
    require_device(t, name);
}

void check_alibi_shape(const kcr_tensor* alibi, int64_t b, int64_t h, int32_t& alibi_b) {
    alibi_b = 0;
    if (!alibi) return;
    if (alibi->dtype != KCR_FLOAT32 || !is_contiguous(*alibi)) {
        throw value_error("alibi must be contiguous float32");
    }
    if (alibi->ndim == 1 && alibi->shape[0] == h) {
        alibi_b = 0;
    } else if (alibi->ndim == 2 && alibi->shape[0] == b && alibi->shape[1] == h) {
        alibi_b = static_cast<int32_t>(h);
    } else {
        throw value_error("alibi must have shape [H] or [B,H]");
    }
    require_device(alibi, "alibi");
}

// gradient_scale = scale / keep (host/backward.rs:159-160): dS is formed with the
// masked dP and the keep-scaled delta, so its 1 / keep rides on dQ and dK.
void fill_common(BwdParams& prm, const Options& opt, double scale_used, const DropoutArgs& drop) {
    set_dropout(prm, drop);
    prm.window_left = opt.window_left;
    prm.window_right = opt.window_right;
    prm.alibi_causal = opt.alibi_causal;
    prm.scale_log2 = opt.scale * kLog2e;
    prm.tanh_scale = opt.tanh_scale;
    prm.scale_eff_log2 = opt.scale_eff * kLog2e;
    prm.grad_scale = static_cast<float>(scale_used) / drop.keep;
}

}  // namespace
}  // namespace kcr

using namespace kcr;
using namespace kcr::attn;

extern "C" int kcr_flash_bwd_preprocess(const kcr_tensor* dout, const kcr_tensor* out, double p_dropout,
                                        const kcr_tensor* delta, void* stream) {
    return guarded([&] {
        if (!(p_dropout >= 0.0 && p_dropout < 1.0)) throw value_error("p_dropout must be in [0, 1) as float32");
        check_qkv(dout, "dout", 4);
        check_qkv(out, "out", 4);
        if (shape_of(*dout) != shape_of(*out) || dout->dtype != out->dtype) {
            throw value_error("dout and out must share shape, dtype and device");
        }
        const int64_t B = out->shape[0], S = out->shape[1], H = out->shape[2], D = out->shape[3];
        if (B <= 0 || H <= 0 || B > 65535 || H > 65535 || S < 0 || S > INT32_MAX - 127 || D < 8 ||
            D > 256 || D % 8 != 0) {
            throw value_error("unsupported backward tensor dimensions");
        }
        const int64_t rounded = (S + 127) / 128 * 128;
        check_f32_tensor(delta, {B, H, rounded}, "delta");
        for (auto* t : {dout, out}) require_device(t, "dout/out");
        if (S == 0) return;
        auto s = static_cast<hipStream_t>(stream);
        // Packed copies of rows the kernel cannot read as 16-byte vectors (host/layout.rs:46-125).
        Staged sd_(dout, s, true), so_(out, s, true);
        dout = sd_.get();
        out = so_.get();
        const int lanes = D <= 64 ? 8 : (D <= 128 ? 16 : 32);
        const int64_t rows = B * H * rounded;
        const int64_t blocks = rows / (256 / lanes);
        const float keep = 1.0f - static_cast<float>(p_dropout);
        auto go = [&](auto tag) {
            using T = decltype(tag);
            bwd_preprocess_kernel<T, false><<<static_cast<unsigned>(blocks), 256, 0, s>>>(
                static_cast<const uint16_t*>(dout->data), static_cast<const uint16_t*>(out->data),
                static_cast<float*>(delta->data), nullptr, dout->strides[0], dout->strides[1],
                dout->strides[2], out->strides[0], out->strides[1], out->strides[2], H * rounded,
                rounded, static_cast<int>(S), static_cast<int>(rounded), static_cast<int>(H),
                static_cast<int>(D), lanes, keep, S);
        };
        if (out->dtype == KCR_BFLOAT16) go(bf16_t{}); else go(f16_t{});
        check_launch("launch bwd_preprocess");
    });
}

namespace {
// Head size the backward kernels run at: the tiled kernels' 64, 128 or 256,
// the next one up. Padding 160..224 to 256 runs 1.14-1.6x the matrix work on
// the tiled kernels at ~590 TFLOP/s, against ~110 TFLOP/s for the general
// kernels at the unpadded size.
int64_t bwd_work_dim(int64_t D) { return D <= 64 ? 64 : D <= 128 ? 128 : 256; }
}  // namespace

extern "C" int64_t kcr_flash_bwd_workspace_bytes(int64_t, int64_t, int64_t, int64_t) { return 0; }

extern "C" int kcr_flash_bwd(const kcr_tensor* q, const kcr_tensor* k, const kcr_tensor* v,
                             const kcr_tensor* dout, const kcr_tensor* lse, const kcr_tensor* delta,
                             const kcr_tensor* alibi, int has_scale, double scale, int causal,
                             int64_t window_left, int64_t window_right, double softcap, const kcr_dropout* dropout,
                             const kcr_tensor* dq, const kcr_tensor* dk, const kcr_tensor* dv,
                             void* workspace, int64_t workspace_bytes, void* stream) {
    (void)workspace;
    (void)workspace_bytes;
    return guarded([&] {
        check_qkv(q, "q", 4);
        check_qkv(k, "k", 4);
        check_qkv(v, "v", 4);
        check_qkv(dout, "dout", 4);
        if (k->dtype != q->dtype || v->dtype != q->dtype || dout->dtype != q->dtype) {
            throw value_error("backward inputs must share q's dtype and device");
        }
        const int64_t B = q->shape[0], Sq = q->shape[1], H = q->shape[2], D = q->shape[3];
        const int64_t Sk = k->shape[1], Hk = k->shape[2];
        if (shape_of(*dout) != shape_of(*q) || shape_of(*k) != shape_of(*v) || k->shape[0] != B ||
            k->shape[3] != D) {
            throw value_error("inconsistent backward input shapes");
        }
        if (B <= 0 || H <= 0 || B > 65535 || H > 65535 || Hk <= 0 || H % Hk != 0 || D < 8 || D > 256 ||
            D % 8 != 0 || Sq < 0 || Sq > INT32_MAX - 127 || Sk < 0 || Sk > INT32_MAX - 256) {
            throw value_error("unsupported backward dimensions");
        }
        const int64_t rounded = (Sq + 127) / 128 * 128;
        check_f32_tensor(lse, {B, H, Sq}, "lse");
        check_f32_tensor(delta, {B, H, rounded}, "delta");
        int32_t alibi_b = 0;
        check_alibi_shape(alibi, B, H, alibi_b);
        if ((dk == nullptr) != (dv == nullptr)) throw value_error("dk and dv must be given together");
        check_grad(dq, q, "dq");
        check_grad(dk, k, "dk");
        check_grad(dv, v, "dv");
        for (auto* t : {q, k, v, dout}) require_device(t, "q/k/v/dout");
        auto s = static_cast<hipStream_t>(stream);
        // Packed copies of inputs the tile loads cannot read (host/layout.rs:46-125).
        Staged sq_(q, s, true), sk_(k, s, true, 1, D), sv_(v, s, true, 1, D), sd_(dout, s, true);
        q = sq_.get();
        k = sk_.get();
        v = sv_.get();
        dout = sd_.get();
        const double scale_used = has_scale ? scale : 1.0 / std::sqrt(static_cast<double>(D));
        const Options opt = normalize_options(has_scale, scale, causal, window_left, window_right, softcap, D, Sk);
        const DropoutArgs drop = parse_dropout(dropout, softcap, q);
        if (Sq == 0 || Sk == 0) {
            if (dq) zero_u16(dq->data, numel(*dq), s);
            if (dk) zero_u16(dk->data, numel(*dk), s);
            if (dv) zero_u16(dv->data, numel(*dv), s);
            return;
        }
        // Head sizes other than 64, 128 and 256 run on the tiled kernels through
        // zero-padded copies (bwd_work_dim): the zero columns add nothing to any
        // dot product, and the gradients' first D columns are copied back.
        const int64_t DK = bwd_work_dim(D);
        const bool pad = DK != D && D % 8 == 0;
        Padded pq(pad ? q : nullptr, DK, s, true), pk(pad ? k : nullptr, DK, s, true),
            pv(pad ? v : nullptr, DK, s, true), pdo(pad ? dout : nullptr, DK, s, true);
        Padded pdq(pad ? dq : nullptr, DK, s, false), pdk(pad ? dk : nullptr, DK, s, false),
            pdv(pad ? dv : nullptr, DK, s, false);
        if (pad) {
            q = pq.get();
            k = pk.get();
            v = pv.get();
            dout = pdo.get();
            if (dq) dq = pdq.get();
            if (dk) dk = pdk.get();
            if (dv) dv = pdv.get();
        }
        BwdParams prm{};
        prm.q = q->data; prm.k = k->data; prm.v = v->data; prm.dout = dout->data;
        prm.lse = static_cast<const float*>(lse->data);
        prm.delta = static_cast<const float*>(delta->data);
        prm.dq = dq ? dq->data : nullptr;
        prm.dk = dk ? dk->data : nullptr;
        prm.dv = dv ? dv->data : nullptr;
        prm.alibi = alibi ? static_cast<const float*>(alibi->data) : nullptr;
        prm.q_b = q->strides[0]; prm.q_s = q->strides[1]; prm.q_h = q->strides[2];
        prm.k_b = k->strides[0]; prm.k_s = k->strides[1]; prm.k_h = k->strides[2];
        prm.v_b = v->strides[0]; prm.v_s = v->strides[1]; prm.v_h = v->strides[2];
        prm.do_b = dout->strides[0]; prm.do_s = dout->strides[1]; prm.do_h = dout->strides[2];
        if (dq) { prm.dq_b = dq->strides[0]; prm.dq_s = dq->strides[1]; prm.dq_h = dq->strides[2]; }
        if (dk) { prm.dk_b = dk->strides[0]; prm.dk_s = dk->strides[1]; prm.dk_h = dk->strides[2]; }
        if (dv) { prm.dv_b = dv->strides[0]; prm.dv_s = dv->strides[1]; prm.dv_h = dv->strides[2]; }
        prm.lse_b = H * Sq; prm.lse_h = Sq;
        prm.delta_b = H * rounded; prm.delta_h = rounded;
        prm.batch = static_cast<int32_t>(B);
        prm.heads = static_cast<int32_t>(H);
        prm.kv_heads = static_cast<int32_t>(Hk);
        prm.gqa = static_cast<int32_t>(H / Hk);
        prm.seqlen_q = static_cast<int32_t>(Sq);
        prm.seqlen_k = static_cast<int32_t>(Sk);
        prm.head_dim = static_cast<int32_t>(pad ? DK : D);
        prm.alibi_b = alibi_b;
        fill_common(prm, opt, scale_used, drop);
        const int bucket = static_cast<int>(((pad ? DK : D) + 31) / 32 * 32);
        launch_bwd<false>(prm, q->dtype, bucket, opt.tanh_scale > 0.0f || alibi, dq != nullptr, dk != nullptr, s);
        pdq.copy_out();
        pdk.copy_out();
        pdv.copy_out();
    });
}

extern "C" int64_t kcr_flash_varlen_bwd_workspace_bytes(int64_t, int64_t, int64_t, int64_t) { return 0; }

extern "C" int kcr_flash_varlen_bwd(const kcr_tensor* q, const kcr_tensor* k, const kcr_tensor* v,
                                    const kcr_tensor* dout, const kcr_tensor* out, const kcr_tensor* lse,
                                    const kcr_tensor* cu_seqlens_q, const kcr_tensor* cu_seqlens_k,
                                    const kcr_tensor* alibi, int has_scale, double scale, int causal,
                                    int64_t window_left, int64_t window_right, double softcap, const kcr_dropout* dropout,
                                    int64_t max_seqlen_q, int64_t max_seqlen_k, int zero_tensors,
                                    const kcr_tensor* dq, const kcr_tensor* dk, const kcr_tensor* dv,
                                    const kcr_tensor* delta, void* workspace, int64_t workspace_bytes,
                                    void* stream) {
    (void)workspace;
    (void)workspace_bytes;
    (void)zero_tensors;
    return guarded([&] {
        check_qkv(q, "q", 3);
        check_qkv(k, "k", 3);
        check_qkv(v, "v", 3);
        check_qkv(dout, "dout", 3);
        check_qkv(out, "out", 3);
        if (k->dtype != q->dtype || v->dtype != q->dtype || dout->dtype != q->dtype || out->dtype != q->dtype ||
            shape_of(*k) != shape_of(*v) || shape_of(*dout) != shape_of(*q) || shape_of(*out) != shape_of(*q) ||
            k->shape[2] != q->shape[2]) {
            throw value_error("inconsistent packed backward inputs");
        }
        if (!cu_seqlens_q || cu_seqlens_q->ndim != 1 || cu_seqlens_q->shape[0] < 2) {
            throw value_error("cu_seqlens_q must have shape [batch + 1]");
        }
        const int64_t batch = cu_seqlens_q->shape[0] - 1;
        const int64_t Tq = q->shape[0], H = q->shape[1], D = q->shape[2];
        const int64_t Hk = k->shape[1];
        if (batch <= 0 || batch > 65535 || H <= 0 || H > 65535 || Hk <= 0 || H % Hk != 0 || D < 8 ||
            D > 256 || D % 8 != 0 || max_seqlen_q < 0 || max_seqlen_k < 0 ||
            max_seqlen_q > INT32_MAX - 256 || max_seqlen_k > INT32_MAX - 256 || Tq > INT32_MAX) {
            throw value_error("unsupported packed backward dimensions");
        }
        for (auto* t : {cu_seqlens_q, cu_seqlens_k}) {
            if (!t || t->dtype != KCR_INT32 || t->ndim != 1 || t->shape[0] != batch + 1 || !is_contiguous(*t)) {
                throw value_error("cu_seqlens must be contiguous int32 [B+1]");
            }
            require_device(t, "cu_seqlens");
        }
        check_f32_tensor(lse, {H, Tq}, "softmax_lse");
        check_f32_tensor(delta, {H, Tq + 128 * batch}, "delta");
        int32_t alibi_b = 0;
        check_alibi_shape(alibi, batch, H, alibi_b);
        if (!dq || !dk || !dv) throw value_error("dq, dk and dv are required");
        check_grad(dq, q, "dq");
        check_grad(dk, k, "dk");
        check_grad(dv, v, "dv");
        for (auto* t : {q, k, v, dout, out}) require_device(t, "q/k/v/dout/out");
        auto s = static_cast<hipStream_t>(stream);
        // Packed copies of inputs the tile loads cannot read (host/layout.rs:46-125).
        Staged sq_(q, s, true), sk_(k, s, true, 0, D), sv_(v, s, true, 0, D), sd_(dout, s, true),
            so_(out, s, true);
        q = sq_.get();
        k = sk_.get();
        v = sv_.get();
        dout = sd_.get();
        out = so_.get();
        const double scale_used = has_scale ? scale : 1.0 / std::sqrt(static_cast<double>(D));
        int causal_eff = causal;
        if (max_seqlen_q == 1 && !alibi) causal_eff = 0;
        const Options opt = normalize_options(has_scale, scale, causal_eff, window_left, window_right, softcap,
                                              D, max_seqlen_k);
        const DropoutArgs drop = parse_dropout(dropout, softcap, q);
        // Gradients of keys no query sees, rows of empty sequences and the delta
        // padding are defined as zero.
        zero_u16(dq->data, numel(*dq), s);
        zero_u16(dk->data, numel(*dk), s);
        zero_u16(dv->data, numel(*dv), s);
        zero_f32(static_cast<float*>(delta->data), numel(*delta), s);
        if (Tq == 0 || max_seqlen_q == 0 || max_seqlen_k == 0) return;
        const int lanes = D <= 64 ? 8 : (D <= 128 ? 16 : 32);
        const int64_t rounded = (max_seqlen_q + 127) / 128 * 128;
        const int64_t blocks = batch * H * rounded / (256 / lanes);
        auto go = [&](auto tag) {
            using T = decltype(tag);
            bwd_preprocess_kernel<T, true><<<static_cast<unsigned>(blocks), 256, 0, s>>>(
                static_cast<const uint16_t*>(dout->data), static_cast<const uint16_t*>(out->data),
                static_cast<float*>(delta->data), static_cast<const int32_t*>(cu_seqlens_q->data), 0,
                dout->strides[0], dout->strides[1], 0, out->strides[0], out->strides[1], 0,
                Tq + 128 * batch, static_cast<int>(max_seqlen_q), static_cast<int>(rounded),
                static_cast<int>(H), static_cast<int>(D), lanes, drop.keep, Tq);
        };
        if (q->dtype == KCR_BFLOAT16) go(bf16_t{}); else go(f16_t{});
        check_launch("launch varlen preprocess");
        // Head sizes other than 64, 128 and 256: zero-padded copies for the
        // tiled kernels, as in kcr_flash_bwd; the padded gradients start at zero
        // like the caller's (rows no block writes).
        const int64_t DK = bwd_work_dim(D);
        const bool pad = DK != D && D % 8 == 0;
        Padded pq(pad ? q : nullptr, DK, s, true), pk(pad ? k : nullptr, DK, s, true),
            pv(pad ? v : nullptr, DK, s, true), pdo(pad ? dout : nullptr, DK, s, true);
        Padded pdq(pad ? dq : nullptr, DK, s, false), pdk(pad ? dk : nullptr, DK, s, false),
            pdv(pad ? dv : nullptr, DK, s, false);
        if (pad) {
            q = pq.get();
            k = pk.get();
            v = pv.get();
            dout = pdo.get();
            dq = pdq.get();
            dk = pdk.get();
            dv = pdv.get();
            zero_u16(dq->data, numel(*dq), s);
            zero_u16(dk->data, numel(*dk), s);
            zero_u16(dv->data, numel(*dv), s);
        }
        BwdParams prm{};
        prm.q = q->data; prm.k = k->data; prm.v = v->data; prm.dout = dout->data;
        prm.lse = static_cast<const float*>(lse->data);
        prm.delta = static_cast<const float*>(delta->data);
        prm.dq = dq->data; prm.dk = dk->data; prm.dv = dv->data;
        prm.alibi = alibi ? static_cast<const float*>(alibi->data) : nullptr;
        prm.cu_q = static_cast<const int32_t*>(cu_seqlens_q->data);
        prm.cu_k = static_cast<const int32_t*>(cu_seqlens_k->data);
        prm.total_q = static_cast<int32_t>(Tq);
        prm.total_k = static_cast<int32_t>(k->shape[0]);
        prm.q_s = q->strides[0]; prm.q_h = q->strides[1];
        prm.k_s = k->strides[0]; prm.k_h = k->strides[1];
        prm.v_s = v->strides[0]; prm.v_h = v->strides[1];
        prm.do_s = dout->strides[0]; prm.do_h = dout->strides[1];
        prm.dq_s = dq->strides[0]; prm.dq_h = dq->strides[1];
        prm.dk_s = dk->strides[0]; prm.dk_h = dk->strides[1];
        prm.dv_s = dv->strides[0]; prm.dv_h = dv->strides[1];
        prm.lse_b = 0; prm.lse_h = Tq;
        prm.delta_b = 0; prm.delta_h = Tq + 128 * batch;
        prm.batch = static_cast<int32_t>(batch);
        prm.heads = static_cast<int32_t>(H);
        prm.kv_heads = static_cast<int32_t>(Hk);
        prm.gqa = static_cast<int32_t>(H / Hk);
        prm.seqlen_q = static_cast<int32_t>(max_seqlen_q);
        prm.seqlen_k = static_cast<int32_t>(max_seqlen_k);
        prm.head_dim = static_cast<int32_t>(pad ? DK : D);
        prm.alibi_b = alibi_b;
        fill_common(prm, opt, scale_used, drop);
        const int bucket = static_cast<int>(((pad ? DK : D) + 31) / 32 * 32);
        launch_bwd<true>(prm, q->dtype, bucket, opt.tanh_scale > 0.0f || alibi, true, true, s);
        pdq.copy_out();
        pdk.copy_out();
        pdv.copy_out();
    });
}
