"""FlashAttention-2 v2-style Python API on MI355X, mirroring
flash-attn2-rs/tvm-ffi-ext/flash_attn2_rs/flash_attn_interface.py:

  fwd / bwd / varlen_fwd / varlen_bwd          (interface.py:732-1471)
  flash_attn_func, flash_attn_qkvpacked_func, flash_attn_kvpacked_func,
  flash_attn_varlen_func, flash_attn_varlen_qkvpacked_func,
  flash_attn_varlen_kvpacked_func              (interface.py:1707-1903)

Same argument names, defaults, return lists and error kinds for the validation
that matters on this path (dtype, device, shapes, head size, GQA divisibility).

Dropout uses the reference's Philox4x32-7 mask stream keyed by a CUDA int64 [2]
RNG-state tensor [seed, offset], returned by the forward and passed to the
backward. The reference reserves those values with
`torch.Generator.philox_state` (Torch >= 2.14). On older Torch this build
reserves them from the generator's seed and Philox offset, advancing the offset
by the same increment, so a generator in the same state gives the reference's
[seed, offset] and masks (under graph capture on older Torch, fresh values
drawn with `torch.randint`). With return_softmax the forward also returns the diagnostic
probabilities [B, H, ceil128(Sq), ceil128(Sk)]: the softmax probability of each
visible element, its sign bit set where dropout drops it.
"""

from __future__ import annotations

import math

import torch

from ._ops import ops


def _cpu_dispatch(op):
    raise NotImplementedError(f"flash_attn2_rs::{op} has no CPU implementation")


def _check_dropout(p, softcap=0.0):
    p = float(p)
    if not math.isfinite(p) or not 0.0 <= p < 1.0:
        raise RuntimeError("p_dropout must be finite and in [0, 1) as float32")
    if p > 0.0 and float(softcap) > 0.0:
        raise RuntimeError("Softcapping does not support dropout for now")
    return p


def _descriptor_values(generator, increment):
    """A Philox reservation of `increment` from a CUDA generator as (seed, offset,
    intragraph, captured). With torch.Generator.philox_state (Torch >= 2.14) this
    is that reservation, made atomically by Torch, as the reference makes it
    (flash_attn_interface.py:53-73). Without it, outside graph capture, the same
    values come from the generator's seed and Philox offset, which then advances
    by the increment rounded to a multiple of 4, as Torch's own reservation does.
    Under graph capture on older Torch no capture-safe reservation exists, and
    fresh values are drawn from the generator with torch.randint instead."""
    reserve = getattr(generator, "philox_state", None)
    if reserve is not None:
        seed, offset, intragraph = reserve(increment)
        captured = seed.is_cuda
        return (seed.data_ptr() if captured else seed.item(), offset.data_ptr() if captured else offset.item(),
                intragraph.item(), int(captured))
    if torch.cuda.is_current_stream_capturing():
        return None
    seed, offset = generator.initial_seed(), generator.get_offset()
    generator.set_offset(offset + (increment + 3) // 4 * 4)
    return seed, offset, 0, 0


def _reserve_rng_state(q, batch, heads, gen=None):
    """CUDA int64 [seed, offset] reserving FlashAttention-2's batch*heads*32 Philox
    increment from `gen` (default: the device's CUDA generator), without a host
    synchronisation (flash_attn_interface.py:36-44)."""
    if gen is not None and not isinstance(gen, torch.Generator):
        raise RuntimeError("gen must be a torch.Generator")
    g = gen if gen is not None else torch.cuda.default_generators[q.device.index or 0]
    if g.device.type != "cuda":
        raise RuntimeError("gen must be a CUDA torch.Generator")
    with torch.cuda.device(q.device):
        values = _descriptor_values(g, int(batch) * int(heads) * 32)
        if values is None:
            return torch.randint(-(2**63), 2**63 - 1, (2,), device=q.device, dtype=torch.int64, generator=g)
        seed, offset, intragraph, captured = values
        return ops.rng_state(q, seed, offset, intragraph, bool(captured))


def reserve_rng_state(q, gen=None):
    """Reserve FlashAttention-2's B*H*32 Philox increment and return CUDA int64
    [seed, offset] (flash_attn_interface.py:20-33)."""
    if not isinstance(q, torch.Tensor) or not q.is_cuda or q.ndim != 4:
        raise ValueError("q must be a CUDA tensor of shape [B, S, H, D]")
    if q.shape[0] <= 0 or q.shape[2] <= 0:
        raise ValueError("q must have positive batch and head counts")
    if gen is not None:
        if not isinstance(gen, torch.Generator) or gen.device.type != "cuda":
            raise TypeError("gen must be a CUDA torch.Generator")
        if gen.device.index not in (None, q.device.index):
            raise ValueError("gen must be on q's device")
    return _reserve_rng_state(q, q.shape[0], q.shape[2], gen)


def _new_rng_state(q, gen=None, batch=None, heads=None):
    if batch is None:
        batch, heads = q.shape[0], q.shape[2]
    return _reserve_rng_state(q, batch, heads, gen)


def _check_return_softmax(return_softmax, p):
    if return_softmax and p == 0:
        raise RuntimeError("return_softmax is only supported when p_dropout > 0.0")


def _validate(q, k, v, out, alibi, softcap, *, packed=False):
    rank = 3 if packed else 4
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not isinstance(t, torch.Tensor) or not t.is_cuda or t.ndim != rank:
            raise RuntimeError(f"{name} must be a CUDA tensor of shape [B, S, H, D]")
        if t.dtype not in (torch.float16, torch.bfloat16) or t.dtype != q.dtype:
            raise RuntimeError(
                "FlashAttention only support fp16 and bf16 data type"
                if name == "q"
                else f"query and {'key' if name == 'k' else 'value'} must have the same dtype"
            )
        if t.device != q.device:
            raise RuntimeError("q, k, v must share device")
        if t.stride(-1) != 1:
            raise RuntimeError("Input tensor must have contiguous last dimension")
    if packed:
        b = 1
        h, d = q.shape[-2:]
    else:
        b, _, h, d = q.shape
    if not 0 < b <= 65535 or not 0 < h <= 65535 or d < 8 or d > 256 or d % 8:
        raise RuntimeError(
            "batch and heads must each be in 1..65535 and head size a multiple of 8 in 8..256"
        )
    if (not packed and k.shape[0] != b) or k.shape[-1] != d or k.shape != v.shape:
        raise RuntimeError("k and v must have matching [B, Sk, Hk, D] shapes")
    if k.shape[-2] == 0 or h % k.shape[-2]:
        raise RuntimeError("the number of KV heads must divide the number of query heads")
    if out is not None:
        if (not isinstance(out, torch.Tensor) or out.device != q.device or out.dtype != q.dtype
                or out.shape != q.shape):
            raise RuntimeError("out must match q's shape, dtype and device")
        if out.stride(-1) != 1:
            raise RuntimeError("out must have unit last stride")
    if alibi is not None:
        if not isinstance(alibi, torch.Tensor) or alibi.device != q.device or alibi.dtype != torch.float32:
            raise RuntimeError("alibi_slopes must be float32 on q's device")


def fwd(q, k, v, out=None, alibi_slopes=None, p_dropout=0.0, softmax_scale=None, is_causal=False,
        window_size_left=-1, window_size_right=-1, softcap=0.0, return_softmax=False, gen=None):
    """Return [output, LSE, probabilities, RNG state] (interface.py:732-852)."""
    if q is None or isinstance(q, torch.Tensor) and not q.is_cuda:
        _cpu_dispatch("fwd")
    p = _check_dropout(p_dropout, softcap)
    _check_return_softmax(return_softmax, p)
    _validate(q, k, v, out, alibi_slopes, softcap)
    if softmax_scale is None:
        softmax_scale = 1.0 / (q.shape[-1] ** 0.5)
    if q.shape[1] == 1 and alibi_slopes is None:
        is_causal = False  # v2's single-query convention
    if alibi_slopes is not None:
        alibi_slopes = alibi_slopes.contiguous()
    if out is None:
        out = torch.empty_like(q)
    args = (q, k, v, alibi_slopes, float(softmax_scale), bool(is_causal), int(window_size_left),
            int(window_size_right), float(softcap))
    probabilities = torch.empty(0, device=q.device, dtype=q.dtype)
    if p > 0:
        state = _new_rng_state(q, gen)
        if return_softmax:
            _, lse, probabilities = ops.fwd(*args, p, state, 0, out, True)
        else:
            lse = ops.fwd_lse(*args, p, state, 0, out)
    else:
        state = torch.zeros(2, device=q.device, dtype=torch.int64)
        lse = ops.fwd_lse(*args, out)
    return [out, lse, probabilities, state]


def fwd_explicit(*args):
    return ops.fwd(*args)


def _finish_gradients(actuals, supplied, sources):
    grads = []
    for actual, buf, source in zip(actuals, supplied, sources):
        if buf is None:
            grads.append(actual)
        else:
            with torch.no_grad():
                buf.copy_(actual)
            grads.append(buf)
    return grads


def bwd(dout, q, k, v, out, softmax_lse, dq=None, dk=None, dv=None, alibi_slopes=None,
        p_dropout=0.0, softmax_scale=None, is_causal=False, window_size_left=-1,
        window_size_right=-1, softcap=0.0, deterministic=False, gen=None, rng_state=None):
    """Return [dQ, dK, dV, softmax_d] (interface.py:855-1009). Both the
    deterministic and default paths are deterministic here (fixed-order GQA sums)."""
    if q is None or isinstance(q, torch.Tensor) and not q.is_cuda:
        _cpu_dispatch("bwd")
    p = _check_dropout(p_dropout, softcap)
    _validate(q, k, v, None, alibi_slopes, softcap)
    for name, t in (("dout", dout), ("out", out)):
        if not isinstance(t, torch.Tensor) or t.shape != q.shape or t.device != q.device or t.dtype != q.dtype:
            raise RuntimeError(f"{name} must match q's shape, dtype and device")
    if (not isinstance(softmax_lse, torch.Tensor) or softmax_lse.shape != (q.shape[0], q.shape[2], q.shape[1])
            or softmax_lse.dtype != torch.float32 or not softmax_lse.is_contiguous()):
        raise RuntimeError("softmax_lse must be contiguous float32 [B, H, Sq] on q's device")
    if softmax_scale is None:
        softmax_scale = 1.0 / (q.shape[-1] ** 0.5)
    if alibi_slopes is not None:
        alibi_slopes = alibi_slopes.contiguous()
    if p > 0 and rng_state is None:
        rng_state = _new_rng_state(q, gen)  # as the reference: a fresh reservation
    delta = ops.bwd_preprocess(dout, out, p)
    args = (q, k, v, dout, softmax_lse, delta, alibi_slopes, float(softmax_scale), bool(is_causal),
            int(window_size_left), int(window_size_right), float(softcap), p,
            rng_state if p > 0 else None)
    if deterministic:
        grad_q = ops.bwd_dq(*args)
        grad_k, grad_v = ops.bwd_dkv(*args)
    else:
        grad_q, grad_k, grad_v = ops.bwd_all(*args)
    return [*_finish_gradients((grad_q, grad_k, grad_v), (dq, dk, dv), (q, k, v)), delta]


def _check_varlen_meta(q, cu_seqlens_q, cu_seqlens_k):
    if not isinstance(cu_seqlens_q, torch.Tensor) or cu_seqlens_q.ndim != 1 or cu_seqlens_q.numel() < 2:
        raise RuntimeError("cu_seqlens_q must have shape [batch + 1]")
    batch = cu_seqlens_q.numel() - 1
    if batch > 65535:
        raise RuntimeError("batch must not exceed 65535")
    for name, t in (("cu_seqlens_q", cu_seqlens_q), ("cu_seqlens_k", cu_seqlens_k)):
        if (not isinstance(t, torch.Tensor) or t.shape != (batch + 1,) or t.dtype != torch.int32
                or t.device != q.device or not t.is_contiguous()):
            raise RuntimeError(f"{name} must be contiguous int32 ({batch + 1},) on q's device")
    return batch


def varlen_fwd(q, k, v, cu_seqlens_q, cu_seqlens_k, out=None, seqused_k=None, leftpad_k=None,
               block_table=None, alibi_slopes=None, max_seqlen_q=0, max_seqlen_k=0, p_dropout=0.0,
               softmax_scale=None, zero_tensors=False, is_causal=False, window_size_left=-1,
               window_size_right=-1, softcap=0.0, return_softmax=False, gen=None):
    """Packed forward, returning [out, LSE, probabilities, RNG state] (interface.py:1012-1241)."""
    if q is None or isinstance(q, torch.Tensor) and not q.is_cuda:
        _cpu_dispatch("varlen_fwd")
    if block_table is not None:
        # Paged K/V [pages, page_size, Hk, D] (interface.py:1012-1241 with a block table).
        if softmax_scale is None:
            softmax_scale = 1.0 / (q.shape[-1] ** 0.5)
        output, lse, probabilities = ops.varlen_fwd_explicit(
            q, k, v, cu_seqlens_q, cu_seqlens_k, seqused_k, leftpad_k, alibi_slopes, float(softmax_scale),
            bool(is_causal), int(window_size_left), int(window_size_right), float(softcap), float(p_dropout),
            None, int(max_seqlen_q), int(max_seqlen_k), bool(return_softmax), bool(zero_tensors), block_table)
        if out is not None:
            out.copy_(output)
            output = out
        return [output, lse, probabilities, torch.zeros(2, device=q.device, dtype=torch.int64)]
    p = _check_dropout(p_dropout, softcap)
    _check_return_softmax(return_softmax, p)
    _validate(q, k, v, out, alibi_slopes, softcap, packed=True)
    _check_varlen_meta(q, cu_seqlens_q, cu_seqlens_k)
    if not 0 <= int(max_seqlen_q) <= 2**31 - 128 or not 0 <= int(max_seqlen_k) <= 2**31 - 128:
        raise RuntimeError("maximum sequence lengths must fit nonnegative int32 with rounding")
    if softmax_scale is None:
        softmax_scale = 1.0 / (q.shape[-1] ** 0.5)
    if alibi_slopes is not None:
        alibi_slopes = alibi_slopes.contiguous()
    state = (_new_rng_state(q, gen, cu_seqlens_q.numel() - 1, q.shape[1]) if p > 0
             else torch.zeros(2, device=q.device, dtype=torch.int64))
    output, lse, probabilities = ops.varlen_fwd_explicit(
        q, k, v, cu_seqlens_q, cu_seqlens_k, seqused_k, leftpad_k, alibi_slopes,
        float(softmax_scale), bool(is_causal), int(window_size_left), int(window_size_right),
        float(softcap), p, state if p > 0 else None, int(max_seqlen_q), int(max_seqlen_k),
        bool(return_softmax), bool(zero_tensors))
    if out is not None:
        out.copy_(output)
        output = out
    return [output, lse, probabilities, state]


def varlen_bwd(dout, q, k, v, out, softmax_lse, cu_seqlens_q, cu_seqlens_k, dq=None, dk=None,
               dv=None, alibi_slopes=None, max_seqlen_q=0, max_seqlen_k=0, p_dropout=0.0,
               softmax_scale=None, zero_tensors=False, is_causal=False, window_size_left=-1,
               window_size_right=-1, softcap=0.0, deterministic=False, gen=None, rng_state=None):
    """Packed backward returning [dQ, dK, dV, softmax_d] (interface.py:1244-1471)."""
    if q is None or isinstance(q, torch.Tensor) and not q.is_cuda:
        _cpu_dispatch("varlen_bwd")
    p = _check_dropout(p_dropout, softcap)
    if any(not isinstance(x, torch.Tensor) or x.ndim != 3 for x in (q, k, v)):
        raise RuntimeError("q, k, v must have shape [total_tokens, heads, head_size]")
    _validate(q, k, v, None, alibi_slopes, softcap, packed=True)
    batch = _check_varlen_meta(q, cu_seqlens_q, cu_seqlens_k)
    h = q.shape[1]
    for name, t in (("dout", dout), ("out", out)):
        if (not isinstance(t, torch.Tensor) or t.shape != q.shape or t.device != q.device
                or t.dtype != q.dtype or t.stride(-1) != 1):
            raise RuntimeError(f"{name} must match q's shape, dtype and device with unit last stride")
    if (not isinstance(softmax_lse, torch.Tensor) or softmax_lse.shape != (h, q.shape[0])
            or softmax_lse.dtype != torch.float32 or not softmax_lse.is_contiguous()):
        raise RuntimeError("softmax_lse must be contiguous float32 [H,total_q] on q's device")
    if softmax_scale is None:
        softmax_scale = 1.0 / (q.shape[-1] ** 0.5)
    if alibi_slopes is not None:
        alibi_slopes = alibi_slopes.contiguous()
    if p > 0 and rng_state is None:
        rng_state = _new_rng_state(q, gen, batch, h)
    grad_q, grad_k, grad_v, softmax_d = ops.varlen_bwd_explicit(
        q, k, v, dout, out, softmax_lse, cu_seqlens_q, cu_seqlens_k, alibi_slopes,
        float(softmax_scale), bool(is_causal), int(window_size_left), int(window_size_right),
        float(softcap), p, rng_state if p > 0 else None, int(max_seqlen_q), int(max_seqlen_k),
        bool(zero_tensors))
    return [*_finish_gradients((grad_q, grad_k, grad_v), (dq, dk, dv), (q, k, v)), softmax_d]


def flash_attn_func(q, k, v, dropout_p=0.0, softmax_scale=None, causal=False, window_size=(-1, -1),
                    softcap=0.0, alibi_slopes=None, deterministic=False, return_attn_probs=False):
    """Dense attention with Q/K/V autograd, MQA/GQA and head padding (interface.py:1707)."""
    from ._torch_interface import _DenseAttention

    return _DenseAttention.apply(q, k, v, dropout_p, softmax_scale, causal, window_size, softcap,
                                 alibi_slopes, deterministic, return_attn_probs, 0)


def flash_attn_qkvpacked_func(qkv, dropout_p=0.0, softmax_scale=None, causal=False,
                              window_size=(-1, -1), softcap=0.0, alibi_slopes=None,
                              deterministic=False, return_attn_probs=False):
    """Self-attention with autograd for packed [B, S, 3, H, D] input."""
    from ._torch_interface import _DenseAttention

    return _DenseAttention.apply(qkv, None, None, dropout_p, softmax_scale, causal, window_size,
                                 softcap, alibi_slopes, deterministic, return_attn_probs, 3)


def flash_attn_kvpacked_func(q, kv, dropout_p=0.0, softmax_scale=None, causal=False,
                             window_size=(-1, -1), softcap=0.0, alibi_slopes=None,
                             deterministic=False, return_attn_probs=False):
    """Attention with autograd for Q [B, Sq, H, D] and KV [B, Sk, 2, Hk, D]."""
    from ._torch_interface import _DenseAttention

    return _DenseAttention.apply(q, kv, None, dropout_p, softmax_scale, causal, window_size,
                                 softcap, alibi_slopes, deterministic, return_attn_probs, 2)


def flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                           dropout_p=0.0, softmax_scale=None, causal=False, window_size=(-1, -1),
                           softcap=0.0, alibi_slopes=None, deterministic=False,
                           return_attn_probs=False, block_table=None):
    """Variable-length attention with autograd (interface.py:1800)."""
    from ._torch_interface import _VarlenAttention

    cuk = None if cu_seqlens_k is cu_seqlens_q else cu_seqlens_k
    return _VarlenAttention.apply(q, k, v, cu_seqlens_q, cuk, max_seqlen_q, max_seqlen_k, dropout_p,
                                  softmax_scale, causal, window_size, softcap, alibi_slopes,
                                  deterministic, return_attn_probs, block_table, 0)


def flash_attn_varlen_qkvpacked_func(qkv, cu_seqlens, max_seqlen, dropout_p=0.0, softmax_scale=None,
                                     causal=False, window_size=(-1, -1), softcap=0.0,
                                     alibi_slopes=None, deterministic=False,
                                     return_attn_probs=False):
    """Autograd for variable-length packed [total, 3, H, D] QKV."""
    from ._torch_interface import _VarlenAttention

    return _VarlenAttention.apply(qkv, None, None, cu_seqlens, None, max_seqlen, max_seqlen,
                                  dropout_p, softmax_scale, causal, window_size, softcap,
                                  alibi_slopes, deterministic, return_attn_probs, None, 3)


def flash_attn_varlen_kvpacked_func(q, kv, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                                    dropout_p=0.0, softmax_scale=None, causal=False,
                                    window_size=(-1, -1), softcap=0.0, alibi_slopes=None,
                                    deterministic=False, return_attn_probs=False):
    """Autograd for variable-length Q and packed [total_k, 2, Hk, D] KV."""
    from ._torch_interface import _VarlenAttention

    cuk = None if cu_seqlens_k is cu_seqlens_q else cu_seqlens_k
    return _VarlenAttention.apply(q, kv, None, cu_seqlens_q, cuk, max_seqlen_q, max_seqlen_k,
                                  dropout_p, softmax_scale, causal, window_size, softcap,
                                  alibi_slopes, deterministic, return_attn_probs, None, 2)


def fwd_kvcache(q, kcache, vcache, k=None, v=None, seqlens_k=None, rotary_cos=None, rotary_sin=None,
                cache_batch_idx=None, leftpad_k=None, block_table=None, alibi_slopes=None, out=None,
                softmax_scale=None, is_causal=False, window_size_left=-1, window_size_right=-1, softcap=0.0,
                is_rotary_interleaved=False, num_splits=1):
    """Native cached inference; appends K/V in place and returns [out, LSE]
    (flash_attn_interface.py:1474-1700)."""
    if q is None or isinstance(q, torch.Tensor) and not q.is_cuda:
        _cpu_dispatch("fwd_kvcache")
    return ops.fwd_kvcache(q, kcache, vcache, k, v, seqlens_k, rotary_cos, rotary_sin, cache_batch_idx,
                           leftpad_k, block_table, alibi_slopes, out, softmax_scale, is_causal,
                           window_size_left, window_size_right, softcap, is_rotary_interleaved, num_splits)


def flash_attn_with_kvcache(q, k_cache, v_cache, k=None, v=None, rotary_cos=None, rotary_sin=None,
                            cache_seqlens=None, cache_batch_idx=None, cache_leftpad=None, block_table=None,
                            softmax_scale=None, causal=False, window_size=(-1, -1), softcap=0.0,
                            rotary_interleaved=True, alibi_slopes=None, num_splits=0,
                            return_softmax_lse=False):
    """Cached inference, optionally appending K/V in place; no backward
    (flash_attn_interface.py:1921-1960). Runs as a torch custom op
    (_torch_interface.py:696-758); num_splits = 0 picks the key split count."""
    from ._torch_interface import flash_attn_with_kvcache as implementation

    return implementation(q, k_cache, v_cache, k, v, rotary_cos, rotary_sin, cache_seqlens, cache_batch_idx,
                          cache_leftpad, block_table, softmax_scale, causal, window_size, softcap,
                          rotary_interleaved, alibi_slopes, num_splits, return_softmax_lse)
