// Diagnostic attention probabilities of a dropout forward (`return_softmax`):
// what flash-attn2-rs writes into its `probabilities` output when fwd is called
// with arity 14 and return_softmax = true (src/host/forward/mod.rs:133-199,
// 382-398, 526-540; the write itself is Dropout::apply, src/device/dropout.rs:
// 93-112), and varlen_fwd_explicit with return_softmax (src/host/varlen/mod.rs:
// 201-229, 400-455).
//
// Layout: probs [B, H, ceil128(Sq), ceil128(Sk)] in q's dtype (varlen: B
// sequences, rows and columns local to the sequence, sizes ceil128(max_q) and
// ceil128(max_k)). Element (q, k) with q < Sq and k < Sk that the causal / window
// mask leaves visible holds the softmax probability exp(scale q.k + bias - lse),
// with the sign bit set when the Philox stream drops it; every other element
// (the padding, masked entries) is +0. The reference's kernel writes the
// probabilities scaled by the running row maximum of the key tile being
// processed (a value that depends on its tiling) and encodes the drop decision
// in the same sign bit; here the magnitudes are the final, normalised ones.
//
// One block of 256 threads computes a 64 x 64 tile of the plane: Q and K rows
// staged in LDS, each thread a 4 x 4 sub-tile in fp32 (this is a diagnostic
// output of the size of the score matrix; its cost is the write of that matrix,
// not the dot products). The whole plane is written, padding included, so no
// separate clear is needed.

#include "attention.h"

namespace kcr {
namespace attn {
namespace {

constexpr int kProbTile = 64;
constexpr int kProbMaxD = 256;
constexpr int kProbLdsRow = kProbMaxD + 8;  // elements; (D / 2 + 4) words between rows

// Keep decision for element (q, k) of head bh: byte ((q % 16) / 8 * 2 + k % 2)
// of word (k % 32) / 8 of philox(seed, offset + 32 bh + 4 (q % 8) + (k % 8) / 2,
// q / 16, k / 32) at most the threshold (src/device/dropout.rs:31-121).
__device__ __forceinline__ bool dropout_keep_element(const DropoutState& d, uint32_t bh, uint32_t q, uint32_t k) {
    uint32_t x[4];
    philox4x32_7(d.seed, d.offset + 32ull * bh + 4u * (q % 8u) + (k % 8u) / 2u, q / 16u, k / 32u, x);
    const uint32_t wi = (k % 32u) / 8u;
    const uint32_t w = wi == 0 ? x[0] : wi == 1 ? x[1] : wi == 2 ? x[2] : x[3];
    const uint32_t byte = (w >> (8u * (2u * ((q % 16u) / 8u) + (k & 1u)))) & 255u;
    return byte <= d.threshold;
}

template <typename T, bool VARLEN>
__global__ __launch_bounds__(256) void dropout_probabilities_kernel(FwdParams p, uint16_t* probs, int64_t rq,
                                                                    int64_t rk) {
    __shared__ uint32_t qs[kProbTile * kProbLdsRow / 2];
    __shared__ uint32_t ks[kProbTile * kProbLdsRow / 2];
    const int tid = threadIdx.x;
    const int tx = tid % 16, ty = tid / 16;
    const int k0 = blockIdx.x * kProbTile, q0 = blockIdx.y * kProbTile;
    const int bh = blockIdx.z;
    const int b = bh / p.heads, head = bh % p.heads;
    const int kvh = head / p.gqa;

    int sq = p.seqlen_q, sk = p.seqlen_k;
    int64_t qrow0 = 0, krow0 = 0;
    bool ok = true;
    if constexpr (VARLEN) {
        const VarSeq vs = varlen_seq(p, b);
        ok = vs.ok;
        sq = vs.sq;
        sk = vs.sk;
        qrow0 = vs.qs;
        krow0 = vs.k_row0;
    }
    uint16_t* dst = probs + (static_cast<int64_t>(bh) * rq + q0 + 4 * ty) * rk + k0 + 4 * tx;
    if (!ok || q0 >= sq || k0 >= sk) {
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<uint2*>(dst + i * rk) = uint2{0u, 0u};
        return;  // block-uniform: no barrier follows for this block
    }

    const uint16_t* qbase;
    const uint16_t* kbase;
    if constexpr (VARLEN) {
        qbase = static_cast<const uint16_t*>(p.q) + qrow0 * p.q_s + head * p.q_h;
        kbase = static_cast<const uint16_t*>(p.k) + krow0 * p.k_s + kvh * p.k_h;
    } else {
        qbase = static_cast<const uint16_t*>(p.q) + b * p.q_b + head * p.q_h;
        kbase = static_cast<const uint16_t*>(p.k) + b * p.k_b + kvh * p.k_h;
    }
    // Stage 64 rows of Q and K (pairs of elements; rows past the end as zero).
    const int D = p.head_dim;
    const int pairs = D / 2;
    for (int i = tid; i < kProbTile * pairs; i += 256) {
        const int r = i / pairs, c = i - r * pairs;
        const int qr = q0 + r, kr = k0 + r;
        qs[r * (kProbLdsRow / 2) + c] =
            qr < sq ? *reinterpret_cast<const uint32_t*>(qbase + static_cast<int64_t>(qr) * p.q_s + 2 * c) : 0u;
        ks[r * (kProbLdsRow / 2) + c] =
            kr < sk ? *reinterpret_cast<const uint32_t*>(kbase + static_cast<int64_t>(kr) * p.k_s + 2 * c) : 0u;
    }
    __syncthreads();

    float acc[4][4] = {};
    for (int c = 0; c < pairs; ++c) {
        float qa[4], qb[4], ka[4], kb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t w = qs[(4 * ty + i) * (kProbLdsRow / 2) + c];
            qa[i] = Elem<T>::to_f32(w & 0xffffu);
            qb[i] = Elem<T>::to_f32(w >> 16);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t w = ks[(4 * tx + j) * (kProbLdsRow / 2) + c];
            ka[j] = Elem<T>::to_f32(w & 0xffffu);
            kb[j] = Elem<T>::to_f32(w >> 16);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(qa[i], ka[j], __builtin_fmaf(qb[i], kb[j], acc[i][j]));
        }
    }

    const DropoutState drop = dropout_state(p);
    const float slope_log2 = p.alibi ? p.alibi[b * p.alibi_b + head] * kLog2e : 0.0f;
    const float* lse = p.lse + b * p.lse_b + head * p.lse_h + (VARLEN ? qrow0 : 0);
    const int off = sk - sq;
    const int wl = p.window_left, wr = p.window_right;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = q0 + 4 * ty + i;
        const float lse2 = row < sq ? lse[row] * kLog2e : 0.0f;
        uint32_t h[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int col = k0 + 4 * tx + j;
            const bool visible = row < sq && col < sk && !(wr >= 0 && col > row + off + wr) &&
                                 !(wl >= 0 && col < row + off - wl);
            uint32_t bits = 0;
            if (visible) {
                float x = acc[i][j] * p.scale_log2;
                if (p.alibi) {
                    x += p.alibi_causal ? slope_log2 * static_cast<float>(col)
                                        : -slope_log2 * fabsf(static_cast<float>(row + off - col));
                }
                bits = Elem<T>::from_f32(exp2f(x - lse2));
                if (!dropout_keep_element(drop, static_cast<uint32_t>(bh), static_cast<uint32_t>(row),
                                          static_cast<uint32_t>(col))) {
                    bits |= 0x8000u;
                }
            }
            h[j] = bits;
        }
        *reinterpret_cast<uint2*>(dst + i * rk) = uint2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
    }
}

}  // namespace

void launch_dropout_probabilities(const FwdParams& prm, bool varlen, int dtype, void* probs, int64_t rq,
                                  int64_t rk, hipStream_t s) {
    if (rq == 0 || rk == 0) return;
    const dim3 grid(static_cast<unsigned>(rk / kProbTile), static_cast<unsigned>(rq / kProbTile),
                    static_cast<unsigned>(static_cast<int64_t>(prm.batch) * prm.heads));
    auto* out = static_cast<uint16_t*>(probs);
    auto go = [&](auto tag) {
        using T = decltype(tag);
        if (varlen) {
            dropout_probabilities_kernel<T, true><<<grid, 256, 0, s>>>(prm, out, rq, rk);
        } else {
            dropout_probabilities_kernel<T, false><<<grid, 256, 0, s>>>(prm, out, rq, rk);
        }
    };
    if (dtype == KCR_BFLOAT16) {
        go(bf16_t{});
    } else {
        go(f16_t{});
    }
    check_launch("launch dropout_probabilities");
}

}  // namespace attn
}  // namespace kcr
