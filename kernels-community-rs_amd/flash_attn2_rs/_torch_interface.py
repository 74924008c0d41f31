"""Torch custom ops and autograd Functions behind flash_attn_func /
flash_attn_varlen_func, mirroring flash-attn2-rs/tvm-ffi-ext/flash_attn2_rs/
_torch_interface.py:19-555: head sizes that are not a multiple of 8 are
zero-padded, QKV / KV packings are unbound, and the native forward / backward run
as opaque custom ops with fake (meta) implementations for torch.compile."""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from ._ops import check_cache_append, ops
from ._ops import torch_add_op_namespace_prefix as add_op_namespace_prefix
from .flash_attn_interface import bwd, fwd, varlen_bwd, varlen_fwd


def _custom_op(name):
    return torch.library.custom_op(add_op_namespace_prefix(name), mutates_args=(), device_types="cuda")


@_custom_op("_dense_forward")
def _dense_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, causal: bool,
                   left: int, right: int, softcap: float, slopes: Optional[torch.Tensor],
                   dropout_p: float, return_probs: bool
                   ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    out, lse, probs, rng_state = fwd(q, k, v, alibi_slopes=slopes, p_dropout=dropout_p, softmax_scale=scale,
                                     is_causal=causal, window_size_left=left, window_size_right=right,
                                     softcap=softcap, return_softmax=return_probs)
    return out, lse, probs, rng_state


def _round128(n):
    return (n + 127) // 128 * 128


@_dense_forward.register_fake
def _(q, k, v, scale, causal, left, right, softcap, slopes, dropout_p, return_probs):
    b, sq, h, _ = q.shape
    p_shape = (b, h, _round128(sq), _round128(k.shape[1])) if return_probs else (0,)
    return (torch.empty_like(q), q.new_empty((b, h, sq), dtype=torch.float32), q.new_empty(p_shape),
            q.new_empty((2,), dtype=torch.int64))


@_custom_op("_dense_backward")
def _dense_backward(dout: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    out: torch.Tensor, lse: torch.Tensor, scale: float, causal: bool, left: int,
                    right: int, softcap: float, slopes: Optional[torch.Tensor],
                    deterministic: bool, dropout_p: float,
                    rng_state: Optional[torch.Tensor]) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    dq, dk, dv, _ = bwd(dout, q, k, v, out, lse, alibi_slopes=slopes, p_dropout=dropout_p,
                        softmax_scale=scale, is_causal=causal, window_size_left=left,
                        window_size_right=right, softcap=softcap, deterministic=deterministic,
                        rng_state=rng_state)
    return dq, dk, dv


@_dense_backward.register_fake
def _(dout, q, k, v, out, lse, scale, causal, left, right, softcap, slopes, deterministic, dropout_p,
      rng_state):
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


def _pad(dim, *tensors):
    if dim % 8:
        return tuple(torch.nn.functional.pad(x, (0, 8 - dim % 8)) for x in tensors)
    return tuple(x.contiguous() if x.stride(-1) != 1 else x for x in tensors)


class _DenseAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, dropout_p, softmax_scale, causal, window_size, softcap,
                alibi_slopes, deterministic, return_attn_probs, packing):
        if packing == 3:
            if q.ndim != 5 or q.shape[2] != 3:
                raise ValueError("qkv must have shape [B, S, 3, H, D]")
            q, k, v = q.unbind(2)
        elif packing == 2:
            if k.ndim != 5 or k.shape[2] != 2:
                raise ValueError("kv must have shape [B, Sk, 2, Hk, D]")
            k, v = k.unbind(2)
        if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
            raise ValueError("q, k, v must have shape [B, S, H, D]")
        dim = q.shape[-1]
        if not 0 < dim <= 256:
            raise ValueError("head size must be in 1..256")
        scale = dim ** -0.5 if softmax_scale is None else float(softmax_scale)
        q, k, v = _pad(dim, q, k, v)
        left, right = window_size
        out, lse, probs, rng_state = _dense_forward(q, k, v, scale, bool(causal), int(left), int(right),
                                                    float(softcap), alibi_slopes, float(dropout_p),
                                                    bool(return_attn_probs and float(dropout_p) > 0))
        ctx.save_for_backward(q, k, v, out, lse, alibi_slopes, rng_state)
        ctx.options = (scale, bool(causal), int(left), int(right), float(softcap), bool(deterministic),
                       float(dropout_p))
        ctx.dim, ctx.packing = dim, packing
        out = out[..., :dim]
        if return_attn_probs:
            return out, lse, probs
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, dout, *unused):
        q, k, v, out, lse, slopes, rng_state = ctx.saved_tensors
        scale, causal, left, right, cap, deterministic, dropout_p = ctx.options
        (dout,) = _pad(ctx.dim, dout)
        dq, dk, dv = _dense_backward(dout, q, k, v, out, lse, scale, causal, left, right, cap,
                                     slopes, deterministic, dropout_p,
                                     rng_state if dropout_p > 0 else None)
        dq, dk, dv = (x[..., : ctx.dim] for x in (dq, dk, dv))
        if ctx.packing == 3:
            grads = (torch.stack((dq, dk, dv), dim=2), None, None)
        elif ctx.packing == 2:
            grads = (dq, torch.stack((dk, dv), dim=2), None)
        else:
            grads = (dq, dk, dv)
        return (*grads, *(None,) * 9)


@_custom_op("_varlen_forward")
def _varlen_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cuq: torch.Tensor,
                    cuk: torch.Tensor, max_q: int, max_k: int, scale: float, causal: bool,
                    left: int, right: int, softcap: float, slopes: Optional[torch.Tensor],
                    dropout_p: float, return_probs: bool
                    ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    out, lse, probs, rng_state = varlen_fwd(q, k, v, cuq, cuk, max_seqlen_q=max_q, max_seqlen_k=max_k,
                                            p_dropout=dropout_p, softmax_scale=scale, is_causal=causal,
                                            window_size_left=left, window_size_right=right,
                                            softcap=softcap, alibi_slopes=slopes, return_softmax=return_probs)
    return out, lse, probs, rng_state


@_varlen_forward.register_fake
def _(q, k, v, cuq, cuk, max_q, max_k, scale, causal, left, right, softcap, slopes, dropout_p,
      return_probs):
    total, h, _ = q.shape
    p_shape = (cuq.shape[0] - 1, h, _round128(max_q), _round128(max_k)) if return_probs else (0,)
    return (torch.empty_like(q), q.new_empty((h, total), dtype=torch.float32), q.new_empty(p_shape),
            q.new_empty((2,), dtype=torch.int64))


@_custom_op("_varlen_backward")
def _varlen_backward(dout: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     out: torch.Tensor, lse: torch.Tensor, cuq: torch.Tensor, cuk: torch.Tensor,
                     max_q: int, max_k: int, scale: float, causal: bool, left: int, right: int,
                     softcap: float, slopes: Optional[torch.Tensor], dropout_p: float,
                     rng_state: Optional[torch.Tensor]) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    dq, dk, dv, _ = varlen_bwd(dout, q, k, v, out, lse, cuq, cuk, alibi_slopes=slopes,
                               max_seqlen_q=max_q, max_seqlen_k=max_k, p_dropout=dropout_p,
                               softmax_scale=scale, is_causal=causal, window_size_left=left,
                               window_size_right=right, softcap=softcap, rng_state=rng_state)
    return dq, dk, dv


@_varlen_backward.register_fake
def _(dout, q, k, v, out, lse, cuq, cuk, max_q, max_k, scale, causal, left, right, softcap, slopes,
      dropout_p, rng_state):
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


class _VarlenAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, cuq, cuk, max_q, max_k, dropout_p, softmax_scale, causal,
                window_size, softcap, slopes, deterministic, return_probs, block_table, packing):
        ctx.paged = block_table is not None
        if block_table is not None:
            # Paged K/V [pages, page_size, Hk, D]: inference only (no backward).
            if float(dropout_p) > 0.0:
                raise ValueError("paged K/V does not support dropout")
            if q.ndim != 3 or k.ndim != 4 or v.ndim != 4:
                raise ValueError("q must be rank 3; k/v must be rank 4 with block_table, otherwise rank 3")
            left, right = window_size
            cuk = cuq if cuk is None else cuk
            out, lse, _ = ops.varlen_fwd_explicit(q, k, v, cuq, cuk, None, None, slopes, softmax_scale,
                                                  causal, left, right, softcap, 0.0, None, max_q, max_k,
                                                  False, False, block_table)
            if return_probs:
                return out, lse, torch.empty(0, device=q.device, dtype=q.dtype)
            return out
        if cuk is None:
            cuk = cuq
        if packing == 3:
            if q.ndim != 4 or q.shape[1] != 3:
                raise ValueError("qkv must have shape [total, 3, H, D]")
            q, k, v = q.unbind(1)
        elif packing == 2:
            if k.ndim != 4 or k.shape[1] != 2:
                raise ValueError("kv must have shape [total_k, 2, Hk, D]")
            k, v = k.unbind(1)
        if q.ndim != 3 or k.ndim != 3 or v.ndim != 3:
            raise ValueError("q must be rank 3; k/v must be rank 4 with block_table, otherwise rank 3")
        dim = q.shape[-1]
        if not 0 < dim <= 256:
            raise ValueError("head size must be in 1..256")
        scale = dim ** -0.5 if softmax_scale is None else float(softmax_scale)
        q, k, v = _pad(dim, q, k, v)
        left, right = window_size
        out, lse, probs, rng_state = _varlen_forward(q, k, v, cuq, cuk, int(max_q), int(max_k), scale,
                                                     bool(causal), int(left), int(right), float(softcap),
                                                     slopes, float(dropout_p),
                                                     bool(return_probs and float(dropout_p) > 0))
        ctx.save_for_backward(q, k, v, out, lse, cuq, cuk, slopes, rng_state)
        ctx.options = (int(max_q), int(max_k), scale, bool(causal), int(left), int(right), float(softcap),
                       float(dropout_p))
        ctx.dim, ctx.packing = dim, packing
        out = out[..., :dim]
        if return_probs:
            return out, lse, probs
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, dout, *unused):
        if ctx.paged:
            raise RuntimeError("paged K/V (block_table) attention has no backward")
        q, k, v, out, lse, cuq, cuk, slopes, rng_state = ctx.saved_tensors
        max_q, max_k, scale, causal, left, right, cap, dropout_p = ctx.options
        (dout,) = _pad(ctx.dim, dout)
        dq, dk, dv = _varlen_backward(dout, q, k, v, out, lse, cuq, cuk, max_q, max_k, scale,
                                      causal, left, right, cap, slopes, dropout_p,
                                      rng_state if dropout_p > 0 else None)
        dq, dk, dv = (x[..., : ctx.dim] for x in (dq, dk, dv))
        if ctx.packing == 3:
            grads = (torch.stack((dq, dk, dv), dim=1), None, None)
        elif ctx.packing == 2:
            grads = (dq, torch.stack((dk, dv), dim=1), None)
        else:
            grads = (dq, dk, dv)
        return (*grads, *(None,) * 14)


# flash_attn_with_kvcache as custom ops (_torch_interface.py:696-758): the
# appending form declares the caches mutated, the read-only form mutates nothing,
# so torch.compile / functionalization see the in-place cache writes.
def _cached_impl(q, k_cache, v_cache, k, v, cache_seqlens, rotary_cos, rotary_sin, cache_batch_idx,
                 cache_leftpad, block_table, alibi_slopes, softmax_scale, causal, left, right, softcap,
                 rotary_interleaved, num_splits):
    out, lse = ops.fwd_kvcache(q, k_cache, v_cache, k, v, cache_seqlens, rotary_cos, rotary_sin,
                               cache_batch_idx, cache_leftpad, block_table, alibi_slopes, None, softmax_scale,
                               causal, left, right, softcap, rotary_interleaved, num_splits)
    return out.contiguous(), lse


def _cached_fake(q, *args):
    b, sq, h, _ = q.shape
    return torch.empty_like(q, memory_format=torch.contiguous_format), q.new_empty((b, h, sq), dtype=torch.float32)


@torch.library.custom_op(add_op_namespace_prefix("_cached_forward"), mutates_args=("k_cache", "v_cache"),
                         device_types="cuda")
def _cached_forward(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, k: Optional[torch.Tensor],
                    v: Optional[torch.Tensor], cache_seqlens: Optional[torch.Tensor],
                    rotary_cos: Optional[torch.Tensor], rotary_sin: Optional[torch.Tensor],
                    cache_batch_idx: Optional[torch.Tensor], cache_leftpad: Optional[torch.Tensor],
                    block_table: Optional[torch.Tensor], alibi_slopes: Optional[torch.Tensor],
                    softmax_scale: Optional[float], causal: bool, left: int, right: int, softcap: float,
                    rotary_interleaved: bool, num_splits: int) -> Tuple[torch.Tensor, torch.Tensor]:
    return _cached_impl(q, k_cache, v_cache, k, v, cache_seqlens, rotary_cos, rotary_sin, cache_batch_idx,
                        cache_leftpad, block_table, alibi_slopes, softmax_scale, causal, left, right, softcap,
                        rotary_interleaved, num_splits)


@torch.library.custom_op(add_op_namespace_prefix("_cached_forward_readonly"), mutates_args=(),
                         device_types="cuda")
def _cached_forward_readonly(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                             k: Optional[torch.Tensor], v: Optional[torch.Tensor],
                             cache_seqlens: Optional[torch.Tensor], rotary_cos: Optional[torch.Tensor],
                             rotary_sin: Optional[torch.Tensor], cache_batch_idx: Optional[torch.Tensor],
                             cache_leftpad: Optional[torch.Tensor], block_table: Optional[torch.Tensor],
                             alibi_slopes: Optional[torch.Tensor], softmax_scale: Optional[float], causal: bool,
                             left: int, right: int, softcap: float, rotary_interleaved: bool,
                             num_splits: int) -> Tuple[torch.Tensor, torch.Tensor]:
    return _cached_impl(q, k_cache, v_cache, k, v, cache_seqlens, rotary_cos, rotary_sin, cache_batch_idx,
                        cache_leftpad, block_table, alibi_slopes, softmax_scale, causal, left, right, softcap,
                        rotary_interleaved, num_splits)


_cached_forward.register_fake(_cached_fake)
_cached_forward_readonly.register_fake(_cached_fake)


def flash_attn_with_kvcache(q, k_cache, v_cache, k=None, v=None, rotary_cos=None, rotary_sin=None,
                            cache_seqlens=None, cache_batch_idx=None, cache_leftpad=None, block_table=None,
                            softmax_scale=None, causal=False, window_size=(-1, -1), softcap=0.0,
                            rotary_interleaved=True, alibi_slopes=None, num_splits=0, return_softmax_lse=False):
    if k_cache.stride(-1) != 1 or v_cache.stride(-1) != 1:
        raise AssertionError("k_cache / v_cache must have contiguous last dimension")
    q, k, v = (x.contiguous() if x is not None and x.stride(-1) != 1 else x for x in (q, k, v))
    cache_batch_idx, block_table = (x.contiguous() if x is not None and x.stride(-1) != 1 else x
                                    for x in (cache_batch_idx, block_table))
    if isinstance(cache_seqlens, int):
        cache_seqlens = torch.full((q.shape[0],), cache_seqlens, device=q.device, dtype=torch.int32)
    if k is not None and v is None:
        raise RuntimeError("new V is required when new K is supplied")
    capacity = k_cache.shape[1] * (block_table.shape[1] if block_table is not None else 1)
    # Rejected appends must leave the caches (and their versions) untouched, so
    # the checks run before the mutating op is entered.
    check_cache_append(q, k_cache, k, v, cache_seqlens, capacity)
    forward = _cached_forward if k is not None and (k.ndim != 4 or k.shape[1] > 0) else _cached_forward_readonly
    out, lse = forward(q, k_cache, v_cache, k, v, cache_seqlens, rotary_cos, rotary_sin, cache_batch_idx,
                       cache_leftpad, block_table, alibi_slopes,
                       None if softmax_scale is None else float(softmax_scale), bool(causal),
                       int(window_size[0]), int(window_size[1]), float(softcap), bool(rotary_interleaved),
                       int(num_splits))
    return (out, lse) if return_softmax_lse else out
