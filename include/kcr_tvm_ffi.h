/* tvm-ffi packed-function exports of libkcr_hip.so: the symbols the reference's
 * kernel-builder `_ops` module binds, with the reference's positional arguments
 * and results. Each is a thin adapter over the C ABI of include/kcr_hip.h.
 *
 * Signature (flash-attn2-rs/src/host/forward/mod.rs:815-853):
 *   int32_t __tvm_ffi_<name>(void* handle, const TVMFFIAny* args,
 *                            int32_t num_args, TVMFFIAny* result);
 * TVMFFIAny is tvm-ffi's 16-byte {int32 type_index; uint32 small_str_len;
 * 8-byte value} (flash-attn2-rs/src/host/mod.rs:59-66). Tensor arguments may be
 * DLTensor pointers or Tensor objects. Returns 0, or -1 after raising the error
 * in the caller's tvm-ffi runtime (and leaving it in kcr_last_error()).
 *
 * Stream, output allocation, error raising and Array results go through the
 * tvm-ffi runtime loaded in the calling process (TVMFFIEnvGetStream,
 * TVMFFIEnvTensorAlloc, TVMFFIErrorSetRaisedFromCStr, the `ffi.Array` global
 * function), found at call time. Without one, the ops that only write
 * caller-provided tensors run on the null stream, and the ops that return
 * tensors fail with a RuntimeError. */
#ifndef KCR_TVM_FFI_H
#define KCR_TVM_FFI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct TVMFFIAny TVMFFIAny;

#define KCR_TVM_FFI_EXPORT(name) \
    int32_t __tvm_ffi_##name(void* handle, const TVMFFIAny* args, int32_t num_args, TVMFFIAny* result);

/* activation-rs/src/ops.rs:255-265: (out, input) -> None; fatrelu_and_mul
 * takes (out, input, threshold). */
KCR_TVM_FFI_EXPORT(silu_and_mul)
KCR_TVM_FFI_EXPORT(mul_and_silu)
KCR_TVM_FFI_EXPORT(gelu_and_mul)
KCR_TVM_FFI_EXPORT(gelu_tanh_and_mul)
KCR_TVM_FFI_EXPORT(fatrelu_and_mul)
KCR_TVM_FFI_EXPORT(gelu)
KCR_TVM_FFI_EXPORT(gelu_tanh)
KCR_TVM_FFI_EXPORT(gelu_new)
KCR_TVM_FFI_EXPORT(gelu_fast)
KCR_TVM_FFI_EXPORT(gelu_quick)
KCR_TVM_FFI_EXPORT(silu)

/* rmsnorm/src/ops.rs:237-444: rms_norm_forward(y, rstd, x, weight|None, eps,
 * offset, casting_mode) -> None; rms_norm_backward(dx, dw_partial|None,
 * dy|None, x, weight|None, rstd, offset, casting_mode) -> None;
 * rms_norm_reduce_weight_grad(dw, dw_partial) -> None. */
KCR_TVM_FFI_EXPORT(rms_norm_forward)
KCR_TVM_FFI_EXPORT(rms_norm_backward)
KCR_TVM_FFI_EXPORT(rms_norm_reduce_weight_grad)

/* flash-attn2-rs/src/host/forward/mod.rs:52-199, 815-853: fwd(q, k, v,
 * alibi|None, scale|None, causal, wl, wr, softcap[, p, seed|state, offset]
 * [, out]) -> [out, lse]; fwd_lse(..., out) -> lse. Arity 14 (..., p, state,
 * offset, out|None, return_softmax) returns [out, lse, probabilities]; arity 16
 * adds (reserve Function, generator) and arity 18 (seed, offset, intragraph,
 * captured): the generator descriptor is resolved into `state` first. */
KCR_TVM_FFI_EXPORT(fwd)
KCR_TVM_FFI_EXPORT(fwd_lse)
/* host/rng.rs:50-98: rng_state(reference, seed, offset, intragraph, captured)
 * -> int64 [2] Tensor on reference's device. */
KCR_TVM_FFI_EXPORT(rng_state)
/* host/backward.rs:14-757: bwd_preprocess(dout, out, p) -> delta;
 * bwd_dq / bwd_dkv / bwd_all(q, k, v, dout, lse, delta, alibi, scale, causal,
 * left, right, softcap, p, rng_state) -> dq | [dk, dv] | [dq, dk, dv]. */
KCR_TVM_FFI_EXPORT(bwd_preprocess)
KCR_TVM_FFI_EXPORT(bwd_dq)
KCR_TVM_FFI_EXPORT(bwd_dkv)
KCR_TVM_FFI_EXPORT(bwd_all)
/* host/varlen/mod.rs:21-670 (19 arguments; the 20th, a block table, must be
 * None here) -> [out, lse, probabilities]; host/varlen/backward.rs:15-546
 * (19 arguments) -> [dq, dk, dv, delta]. */
KCR_TVM_FFI_EXPORT(varlen_fwd_explicit)
KCR_TVM_FFI_EXPORT(varlen_bwd_explicit)

#undef KCR_TVM_FFI_EXPORT

#ifdef __cplusplus
}
#endif

#endif /* KCR_TVM_FFI_H */
