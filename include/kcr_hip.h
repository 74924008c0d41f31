/*
 * kcr_hip.h -- C ABI of libkcr_hip.so, the MI355X (gfx950) implementation of the
 * kernels-community-rs hot paths: FlashAttention-2 (dense, varlen, backward),
 * RMSNorm and the gated / element-wise activations.
 *
 * Every entry point replaces one tvm-ffi export of the reference. The reference
 * exports take tvm-ffi `Tensor` handles (DLPack tensors); this ABI takes the same
 * information as a plain `kcr_tensor` (data pointer, dtype, shape, element strides,
 * device ordinal). Outputs that the reference allocates through
 * `TVMFFIEnvTensorAlloc` (host/mod.rs:42-74 in flash-attn2-rs) are passed in
 * preallocated by the caller instead; the caller's allocator is the one the
 * reference would have used.
 *
 * Conventions
 *   - Return value: KCR_OK (0) or one of the error kinds below; the message is
 *     available from kcr_last_error() on the calling thread. The kinds mirror the
 *     tvm-ffi error kinds the reference raises (ValueError / TypeError /
 *     RuntimeError), and the messages carry the same substrings the reference
 *     tests match ("out must have shape", "must be even", "same dtype", ...).
 *   - `stream` is a hipStream_t. Every launch is asynchronous on that stream;
 *     no entry point synchronises the host.
 *   - Optional tensors are passed as NULL.
 *   - Tensors must live on the current HIP device.
 */
#ifndef KCR_HIP_H
#define KCR_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum kcr_dtype {
    KCR_FLOAT32 = 0,
    KCR_FLOAT16 = 1,
    KCR_BFLOAT16 = 2,
    KCR_INT32 = 3,
    KCR_INT64 = 4,
    KCR_FLOAT64 = 5,
    KCR_DTYPE_OTHER = 99
};

enum kcr_status {
    KCR_OK = 0,
    KCR_VALUE_ERROR = 1,
    KCR_TYPE_ERROR = 2,
    KCR_RUNTIME_ERROR = 3
};

#define KCR_MAX_DIMS 8

/* A strided device tensor: the DLPack fields the reference reads from a tvm-ffi Tensor. */
typedef struct kcr_tensor {
    void* data;                      /* address of element [0, ..., 0] */
    int32_t dtype;                   /* enum kcr_dtype */
    int32_t ndim;                    /* 0 .. KCR_MAX_DIMS */
    int32_t device;                  /* HIP device ordinal */
    int32_t reserved;                /* must be 0 */
    int64_t shape[KCR_MAX_DIMS];
    int64_t strides[KCR_MAX_DIMS];   /* in elements */
} kcr_tensor;

/* Thread-local message of the last failed call on this thread ("" if none). */
const char* kcr_last_error(void);
/* Library version string. */
const char* kcr_version(void);

/* ------------------------------------------------------------------------ */
/* activation-rs: activation-rs/src/ops.rs:196-265                           */
/* ------------------------------------------------------------------------ */
/* out[..., d] = act(input[..., :d]) * input[..., d:]  (ops.rs:200-217)      */
/* replaces tvm export `silu_and_mul` (activation-rs/src/ops.rs:200, 255)    */
int kcr_silu_and_mul(const kcr_tensor* out, const kcr_tensor* input, void* stream);
/* replaces `mul_and_silu` (ops.rs:204-207, 256): input[..., :d] * silu(input[..., d:]) */
int kcr_mul_and_silu(const kcr_tensor* out, const kcr_tensor* input, void* stream);
/* replaces `gelu_and_mul` (ops.rs:209-212, 257): exact erf GELU */
int kcr_gelu_and_mul(const kcr_tensor* out, const kcr_tensor* input, void* stream);
/* replaces `gelu_tanh_and_mul` (ops.rs:214-217, 258) */
int kcr_gelu_tanh_and_mul(const kcr_tensor* out, const kcr_tensor* input, void* stream);
/* replaces `fatrelu_and_mul` (ops.rs:219-223, 259) */
int kcr_fatrelu_and_mul(const kcr_tensor* out, const kcr_tensor* input, double threshold,
                        void* stream);
/* element-wise: out = act(input). Replace `gelu`, `gelu_tanh`, `gelu_new`,
 * `gelu_fast`, `gelu_quick`, `silu` (ops.rs:225-253, 260-265) */
int kcr_gelu(const kcr_tensor* out, const kcr_tensor* input, void* stream);
int kcr_gelu_tanh(const kcr_tensor* out, const kcr_tensor* input, void* stream);
int kcr_gelu_new(const kcr_tensor* out, const kcr_tensor* input, void* stream);
int kcr_gelu_fast(const kcr_tensor* out, const kcr_tensor* input, void* stream);
int kcr_gelu_quick(const kcr_tensor* out, const kcr_tensor* input, void* stream);
int kcr_silu(const kcr_tensor* out, const kcr_tensor* input, void* stream);

/* ------------------------------------------------------------------------ */
/* rmsnorm: rmsnorm/src/ops.rs:237-444                                       */
/* ------------------------------------------------------------------------ */
/* casting_mode: "llama", "gemma" or "none" (rmsnorm/src/ops.rs:28-37).      */
/* replaces `rms_norm_forward(y, rstd, x, weight, eps, offset, casting_mode)` */
/* (rmsnorm/src/ops.rs:237-265, 442)                                          */
int kcr_rms_norm_forward(const kcr_tensor* y, const kcr_tensor* rstd, const kcr_tensor* x,
                         const kcr_tensor* weight /* nullable */, double eps, double offset,
                         const char* casting_mode, void* stream);
/* replaces `rms_norm_backward(dx, dw_partial, dy, x, weight, rstd, offset, casting_mode)` */
/* (rmsnorm/src/ops.rs:326-380, 443). dy == NULL: the gradient is read from dx   */
/* and overwritten (in place).                                                   */
int kcr_rms_norm_backward(const kcr_tensor* dx, const kcr_tensor* dw_partial /* nullable */,
                          const kcr_tensor* dy /* nullable */, const kcr_tensor* x,
                          const kcr_tensor* weight /* nullable */, const kcr_tensor* rstd,
                          double offset, const char* casting_mode, void* stream);
/* replaces `rms_norm_reduce_weight_grad(dw, dw_partial)` (rmsnorm/src/ops.rs:383-440, 444) */
int kcr_rms_norm_reduce_weight_grad(const kcr_tensor* dw, const kcr_tensor* dw_partial,
                                    void* stream);

/* ------------------------------------------------------------------------ */
/* flash-attn2-rs                                                           */
/* ------------------------------------------------------------------------ */
/* Scalars common to the attention entry points:
 *   has_scale/scale : softmax scale; has_scale == 0 means None (D^-0.5)
 *   causal          : bottom-right aligned causal mask (col > row + Sk - Sq masked)
 *   window_left/right: sliding window, -1 = unbounded (host/forward/mod.rs:310-328)
 *   softcap         : 0 = off; else scores = softcap * tanh(qk * scale / softcap)
 *   alibi           : float32 [H] or [B, H] slopes, nullable
 */

/* Dropout arguments of the attention entry points (NULL = no dropout). p in
 * [0, 1) as float32; p == 0 disables it. The mask is FlashAttention-2's
 * Philox4x32-7 stream (flash-attn2-rs/src/device/dropout.rs:31-121) keyed by
 * (seed, offset): element (query q, key k) of head b * H + h is kept when byte
 * ((q % 16) / 8 * 2 + k % 2) of word (k % 32) / 8 of
 * philox(seed, offset + 32 (b H + h) + 4 (q % 8) + (k % 8) / 2, q / 16, k / 32) is at
 * most floor((1 - p) * 255). With rng_state (a device int64 [2] tensor holding
 * [seed, offset], read by the kernels on the launch stream) the seed and offset
 * fields must be 0 and are ignored (host/forward/mod.rs:91-131). */
typedef struct kcr_dropout {
    double p;
    uint64_t seed;
    uint64_t offset;
    const kcr_tensor* rng_state;  /* nullable */
} kcr_dropout;

/* Dropout RNG state from a generator descriptor. replaces the `rng_state(reference,
 * seed, offset, intragraph, captured)` export (flash-attn2-rs/src/host/rng.rs:13-98,
 * kernel src/device/rng.rs:1-26) and the descriptor step of `fwd` at arities 16
 * and 18 (src/host/forward/mod.rs:132-178, 492-523). Writes [seed, offset] into
 * `state` (contiguous int64 [2] on the device) on `stream`: with captured == 0
 * the values themselves, with captured != 0 the 8-byte values at device
 * addresses `seed` and `offset`, the offset plus `intragraph` (a reservation
 * made under graph capture, resolved at each replay). */
int kcr_flash_rng_state(const kcr_tensor* state, uint64_t seed, uint64_t offset, uint64_t intragraph,
                        int captured, void* stream);

/* Dense forward. replaces `fwd_lse(q,k,v,alibi,scale,causal,wl,wr,softcap,out)`
 * (flash-attn2-rs/src/host/forward/mod.rs:835-853; arities mod.rs:53-61) and `fwd`
 * (mod.rs:815-833); dropout as in mod.rs:73-199 (return_softmax: kcr_flash_fwd_softmax).
 *   q [B,Sq,H,D], k/v [B,Sk,Hk,D] fp16/bf16, last stride 1;
 *   out like q (written), lse float32 contiguous [B,H,Sq] (written). */
int kcr_flash_fwd(const kcr_tensor* q, const kcr_tensor* k, const kcr_tensor* v,
                  const kcr_tensor* alibi, int has_scale, double scale, int causal,
                  int64_t window_left, int64_t window_right, double softcap, const kcr_dropout* dropout,
                  const kcr_tensor* out, const kcr_tensor* lse, void* stream);

/* Dense forward with diagnostic probabilities. replaces `fwd` with arity 14 and
 * return_softmax = true (flash-attn2-rs/src/host/forward/mod.rs:133-199, 382-398,
 * 526-540; kernel write src/device/dropout.rs:93-112). Arguments as kcr_flash_fwd;
 * dropout must have p > 0 and an rng_state tensor. probabilities: contiguous,
 * q's dtype, [B, H, ceil128(Sq), ceil128(Sk)] (written in full): element (q, k)
 * that the mask leaves visible holds exp(scale q.k + bias - lse), its sign bit
 * set when dropout drops it; padding and masked elements are +0. (The
 * reference's magnitudes carry the running maximum of its key tile instead of
 * the final LSE; the sign pattern is the same.) */
int kcr_flash_fwd_softmax(const kcr_tensor* q, const kcr_tensor* k, const kcr_tensor* v,
                          const kcr_tensor* alibi, int has_scale, double scale, int causal,
                          int64_t window_left, int64_t window_right, double softcap, const kcr_dropout* dropout,
                          const kcr_tensor* out, const kcr_tensor* lse, const kcr_tensor* probabilities,
                          void* stream);

/* Varlen forward. replaces the plain (non-paged, non-cached, p == 0) form of
 * `varlen_fwd_explicit(q,k,v,cuq,cuk,seqused_k,leftpad_k,alibi,scale,causal,
 * left,right,softcap,p,state,max_q,max_k,return_softmax,zero_tensors)`
 * (flash-attn2-rs/src/host/varlen/mod.rs:21-670).
 *   q [Tq,H,D], k/v [Tk,Hk,D]; cu_seqlens_q/k int32 [B+1]; seqused_k, leftpad_k
 *   int32 [B] nullable; out like q; lse float32 contiguous [H, Tq]. */
int kcr_flash_varlen_fwd(const kcr_tensor* q, const kcr_tensor* k, const kcr_tensor* v,
                         const kcr_tensor* cu_seqlens_q, const kcr_tensor* cu_seqlens_k,
                         const kcr_tensor* seqused_k, const kcr_tensor* leftpad_k,
                         const kcr_tensor* alibi, int has_scale, double scale, int causal,
                         int64_t window_left, int64_t window_right, double softcap, const kcr_dropout* dropout,
                         int64_t max_seqlen_q, int64_t max_seqlen_k, int zero_tensors,
                         const kcr_tensor* out, const kcr_tensor* lse, void* stream);

/* Varlen forward with diagnostic probabilities. replaces `varlen_fwd_explicit`
 * with return_softmax = true (flash-attn2-rs/src/host/varlen/mod.rs:201-209,
 * 400-455). Arguments as kcr_flash_varlen_fwd; probabilities as for
 * kcr_flash_fwd_softmax with shape [B, H, ceil128(max_seqlen_q),
 * ceil128(max_seqlen_k)], rows and columns local to sequence b. */
int kcr_flash_varlen_fwd_softmax(const kcr_tensor* q, const kcr_tensor* k, const kcr_tensor* v,
                                 const kcr_tensor* cu_seqlens_q, const kcr_tensor* cu_seqlens_k,
                                 const kcr_tensor* seqused_k, const kcr_tensor* leftpad_k,
                                 const kcr_tensor* alibi, int has_scale, double scale, int causal,
                                 int64_t window_left, int64_t window_right, double softcap,
                                 const kcr_dropout* dropout, int64_t max_seqlen_q, int64_t max_seqlen_k,
                                 int zero_tensors, const kcr_tensor* out, const kcr_tensor* lse,
                                 const kcr_tensor* probabilities, void* stream);

/* KV-cache append. replaces `cache_update_explicit(q, kcache, vcache, k, v, lengths,
 * cos, sin, indices, table, interleaved, advance_q)` (flash-attn2-rs/src/host/cache/
 * mod.rs:36-320, kernel src/device/cache.rs:26-330).
 *   New rows k/v [B, Snew, Hk, D] go to cache position seqlens[b] + r of cache batch
 *   cache_batch_idx[b] (or b), or of page block_table[b, position / page] (page =
 *   kcache.shape[1], a multiple of 256). kcache/vcache [batches | pages, rows, Hk, D].
 *   With rotary_cos/sin [positions, rotary_dim / 2] (q's dtype), K is rotated at its
 *   position and q into q_out at seqlens[b] + (advance_q ? r : 0); interleaved pairs
 *   columns (2i, 2i + 1), otherwise (i, i + rotary_dim / 2). q_out may be NULL
 *   without rotary tables. */
int kcr_flash_cache_update(const kcr_tensor* q, const kcr_tensor* kcache, const kcr_tensor* vcache,
                           const kcr_tensor* k, const kcr_tensor* v, const kcr_tensor* seqlens,
                           const kcr_tensor* rotary_cos, const kcr_tensor* rotary_sin,
                           const kcr_tensor* cache_batch_idx, const kcr_tensor* block_table,
                           int interleaved, int advance_q, const kcr_tensor* q_out, void* stream);

/* Attention over a KV cache. replaces the cached mode of `varlen_fwd_explicit`
 * (args 19-23: block_table, cache_batch_idx, new_keys, num_splits, grouped;
 * flash-attn2-rs/src/host/varlen/mod.rs:36-670, device/varlen/mod.rs:60-170,
 * device/varlen/paged.rs, device/varlen/merge.rs).
 *   q [Tq, H, D] packed with cu_seqlens_q int32 [B+1]; sequence b attends to cache
 *   rows [leftpad_k[b], seqused_k[b] + new_keys) (seqused_k: cache lengths before
 *   an append of new_keys rows; NULL: every row of the cache, new_keys ignored)
 *   of cache batch cache_batch_idx[b] (or b), or of pages block_table[b, :]
 *   (int32 [B, max_blocks]; head size 64, 128 or 256). out like q;
 *   lse float32 [H, Tq]. Batched form: cu_seqlens_q NULL, q and out [B, R, H, D]
 *   with any 16-byte aligned row strides (e.g. the grouped decode view of
 *   [B, 1, H*G, D] as [B, G, H, D]) and lse float32 [B, H, R] with unit last
 *   stride; max_seqlen_q is taken as R. Windows are normalised against the cache
 *   capacity.
 *   num_splits > 1 splits each query tile's keys over that many blocks; the fp32
 *   partials go to `workspace` (kcr_flash_fwd_kvcache_workspace_bytes bytes,
 *   16-byte aligned) and a merge kernel writes out/lse. Head sizes other than 64,
 *   128 and 256 run unsplit. */
int64_t kcr_flash_fwd_kvcache_workspace_bytes(int64_t num_splits, int64_t heads, int64_t total_q,
                                              int64_t head_dim);
int kcr_flash_fwd_kvcache(const kcr_tensor* q, const kcr_tensor* kcache, const kcr_tensor* vcache,
                          const kcr_tensor* cu_seqlens_q, const kcr_tensor* seqused_k, int64_t new_keys,
                          const kcr_tensor* leftpad_k, const kcr_tensor* cache_batch_idx,
                          const kcr_tensor* block_table, const kcr_tensor* alibi, int has_scale,
                          double scale, int causal, int64_t window_left, int64_t window_right,
                          double softcap, int64_t max_seqlen_q, int64_t num_splits, void* workspace,
                          int64_t workspace_bytes, const kcr_tensor* out, const kcr_tensor* lse,
                          void* stream);

/* Attention over a KV cache without allocation: kcr_flash_fwd_kvcache with the
 * split partials in a fixed scratch array inside the library instead of a
 * caller workspace. No counterpart in the reference; it is for callers that
 * cannot allocate (code under HIP graph capture, tight decode loops, harnesses
 * that forbid hipMalloc). Each GPU holds one scratch array of
 * kcr_flash_fwd_kvcache_noalloc_scratch_bytes() bytes (64 MiB) for the life of
 * the process, shared by every call on that GPU: calls that overlap on one GPU
 * (concurrent streams) race on it. A call whose num_splits x heads x total_q x
 * (head_dim + 1) x 4 bytes exceed it fails with KCR_VALUE_ERROR. num_splits <= 1
 * uses no scratch. No hipMalloc, hipFree or allocating library call is made;
 * the first call on a device looks up the scratch address there. */
int64_t kcr_flash_fwd_kvcache_noalloc_scratch_bytes(void);
int kcr_flash_fwd_kvcache_noalloc(const kcr_tensor* q, const kcr_tensor* kcache, const kcr_tensor* vcache,
                                  const kcr_tensor* cu_seqlens_q, const kcr_tensor* seqused_k, int64_t new_keys,
                                  const kcr_tensor* leftpad_k, const kcr_tensor* cache_batch_idx,
                                  const kcr_tensor* block_table, const kcr_tensor* alibi, int has_scale,
                                  double scale, int causal, int64_t window_left, int64_t window_right,
                                  double softcap, int64_t max_seqlen_q, int64_t num_splits,
                                  const kcr_tensor* out, const kcr_tensor* lse, void* stream);

/* Backward preprocess. replaces `bwd_preprocess(dout, out, p)`
 * (flash-attn2-rs/src/host/backward.rs:628-737):
 *   delta[b,h,s] = sum_d dout*out * (1-p), float32 [B,H,round128(Sq)], rows >= Sq are 0. */
int kcr_flash_bwd_preprocess(const kcr_tensor* dout, const kcr_tensor* out, double p_dropout,
                             const kcr_tensor* delta, void* stream);

/* Dense backward. replaces `bwd_dq`, `bwd_dkv` and `bwd_all`
 * (flash-attn2-rs/src/host/backward.rs:14-626) with p_dropout == 0.
 *   dq like q, dk/dv like k (GQA-summed, contiguous [B,Sk,Hk,D]); any of dq, dk/dv
 *   may be NULL to skip that component (bwd_dq: dk = dv = NULL; bwd_dkv: dq = NULL).
 *   workspace: float32 scratch, see kcr_flash_bwd_workspace_bytes(). */
int64_t kcr_flash_bwd_workspace_bytes(int64_t batch, int64_t heads, int64_t seqlen_q,
                                      int64_t head_dim);
int kcr_flash_bwd(const kcr_tensor* q, const kcr_tensor* k, const kcr_tensor* v,
                  const kcr_tensor* dout, const kcr_tensor* lse, const kcr_tensor* delta,
                  const kcr_tensor* alibi, int has_scale, double scale, int causal,
                  int64_t window_left, int64_t window_right, double softcap, const kcr_dropout* dropout,
                  const kcr_tensor* dq, const kcr_tensor* dk, const kcr_tensor* dv,
                  void* workspace, int64_t workspace_bytes, void* stream);

/* Varlen backward. replaces `varlen_bwd_explicit` (flash-attn2-rs/src/host/varlen/
 * backward.rs:15-546) with p_dropout == 0. delta float32 [H, Tq + 128*B] is written
 * here (the reference computes it inside the same export, backward.rs:323-346). */
int64_t kcr_flash_varlen_bwd_workspace_bytes(int64_t total_q, int64_t heads, int64_t batch,
                                             int64_t head_dim);
int kcr_flash_varlen_bwd(const kcr_tensor* q, const kcr_tensor* k, const kcr_tensor* v,
                         const kcr_tensor* dout, const kcr_tensor* out, const kcr_tensor* lse,
                         const kcr_tensor* cu_seqlens_q, const kcr_tensor* cu_seqlens_k,
                         const kcr_tensor* alibi, int has_scale, double scale, int causal,
                         int64_t window_left, int64_t window_right, double softcap, const kcr_dropout* dropout,
                         int64_t max_seqlen_q, int64_t max_seqlen_k, int zero_tensors,
                         const kcr_tensor* dq, const kcr_tensor* dk, const kcr_tensor* dv,
                         const kcr_tensor* delta, void* workspace, int64_t workspace_bytes,
                         void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KCR_HIP_H */
