"""`ops` of flash-attn2-rs: the tvm-ffi exports on the hot path, with the reference's
positional signatures and return conventions, backed by libkcr_hip.so.

  fwd(q, k, v, alibi, scale, causal, wl, wr, softcap[, p, seed, offset][, out])
      -> [out, lse]                          host/forward/mod.rs:52-61, 815-833
  fwd(..., p, state, offset, out, return_softmax)
      -> [out, lse, probabilities]           host/forward/mod.rs:133-199, 382-398
  fwd(..., p, state, 0, out, return_softmax, reserve, generator)      (arity 16)
  fwd(..., p, state, 0, out, return_softmax, seed, offset, intragraph, captured)
      (arity 18): the generator descriptor is resolved into `state` first
                                             host/forward/mod.rs:132-178, 492-523
  rng_state(reference, seed, offset, intragraph, captured) -> int64 [2]
                                             host/rng.rs:50-98
  fwd_lse(..., out) -> lse                   host/forward/mod.rs:835-853
  varlen_fwd_explicit(q, k, v, cuq, cuk, seqused_k, leftpad_k, alibi, scale, causal,
      left, right, softcap, p, state, max_q, max_k, return_softmax, zero_tensors)
      -> [out, lse, probabilities]           host/varlen/mod.rs:21-670
  bwd_preprocess(dout, out, p) -> delta      host/backward.rs:628-737
  bwd_dq / bwd_dkv / bwd_all(q, k, v, dout, lse, delta, alibi, scale, causal, left,
      right, softcap, p, rng_state) -> dq | [dk, dv] | [dq, dk, dv]
                                             host/backward.rs:14-626
  varlen_bwd_explicit(q, k, v, dout, out, lse, cuq, cuk, alibi, scale, causal, left,
      right, softcap, p, state, max_q, max_k, zero_tensors) -> [dq, dk, dv, delta]
                                             host/varlen/backward.rs:15-546
  fwd_kvcache(q, kcache, vcache, k, v, seqlens_k, rotary_cos, rotary_sin,
      cache_batch_idx, leftpad_k, block_table, alibi_slopes, out, softmax_scale,
      is_causal, window_size_left, window_size_right, softcap,
      is_rotary_interleaved, num_splits) -> [out, lse]
                                             flash_attn_interface.py:1474-1700,
                                             host/cache/mod.rs:36-320

Outputs the reference allocates with `TVMFFIEnvTensorAlloc` are allocated here with
torch's allocator (the same allocator tvm-ffi forwards to under torch). Inputs
whose rows are not 16-byte aligned are repacked first, as the reference does
with `copy_attention_layout` (host/layout.rs:46-125). Dropout follows the
reference's Philox4x32-7 mask stream, keyed by explicit (seed, offset) or by a
device int64 [2] RNG-state tensor. Diagnostic probabilities (return_softmax)
come from kcr_flash_fwd_softmax / kcr_flash_varlen_fwd_softmax; generator
descriptors (arities 16 and 18, `rng_state`) from kcr_flash_rng_state.
"""

from __future__ import annotations

import ctypes
import math
from types import SimpleNamespace

import numpy as np
import torch

from kcr_native import call, describe, dropout_arg, lib, op_namespace_prefixer, ref, stream_of

torch_add_op_namespace_prefix = op_namespace_prefixer("flash_attn2")


def _rows_aligned(t: torch.Tensor) -> bool:
    if t.data_ptr() % 16:
        return False
    return all(s % 8 == 0 for s, n in zip(t.stride()[:-1], t.shape[:-1]) if n > 1)


def _packed(t):
    """A 16-byte aligned view of `t` with unit last stride (repacked if needed)."""
    if t is None or t.numel() == 0:
        return t
    # Rows of one sequence position must not overlap (e.g. broadcast views).
    if t.stride(-1) == 1 and _rows_aligned(t) and (t.ndim < 3 or t.shape[-3] <= 1
                                                    or t.stride(-3) >= t.shape[-1]):
        return t
    return t.clone(memory_format=torch.contiguous_format)


def _dropout_p(p):
    p = float(p)
    if not (p == p) or not 0.0 <= p < 1.0 or float(np.float32(p)) >= 1.0:
        raise ValueError("p_dropout must be finite and in [0, 1) as float32")
    return p


def _rng_state_ok(state, q):
    return (isinstance(state, torch.Tensor) and state.is_cuda and state.device == q.device
            and state.dtype == torch.int64 and state.shape == (2,) and state.is_contiguous()
            and state.data_ptr() % 8 == 0)


def _round128(n):
    return (int(n) + 127) // 128 * 128


def _scale_args(scale):
    return (0, ctypes.c_double(0.0)) if scale is None else (1, ctypes.c_double(float(scale)))


def _u64(x):
    return ctypes.c_uint64(int(x) & 0xFFFF_FFFF_FFFF_FFFF)


def _resolve_descriptor(state, descriptor, captured):
    """Writes the [seed, offset] of a generator descriptor into `state` on the
    current stream (host/rng.rs:13-47)."""
    seed, offset, intragraph = descriptor
    call("kcr_flash_rng_state", ref(describe(state)), _u64(seed), _u64(offset), _u64(intragraph),
         int(bool(captured)), stream_of(state))


def rng_state(reference, seed, offset, intragraph, captured):
    """CUDA int64 [seed, offset] from a Philox descriptor (host/rng.rs:50-78)."""
    if not isinstance(reference, torch.Tensor) or not reference.is_cuda:
        raise ValueError("RNG state requires a CUDA reference tensor")
    state = torch.empty(2, dtype=torch.int64, device=reference.device)
    _resolve_descriptor(state, (seed, offset, intragraph), captured)
    return state


def _fwd_descriptor(args, n, q, k, p, state, return_softmax):
    """Arities 16 (reserve callback, generator) and 18 (seed, offset, intragraph,
    captured): the descriptor is resolved into the state tensor, which the
    forward then reads (host/forward/mod.rs:132-178, 492-523)."""
    dropout = float(np.float32(p)) > 0.0
    if n == 16:
        if not dropout or state is None:
            raise ValueError("native reservation requires dropout and a state tensor")
    else:
        if (not dropout or q.ndim != 4 or k.ndim != 4 or state is None or q.shape[3] != 64
                or q.shape[1] == 0 or k.shape[1] == 0):
            raise ValueError("RNG descriptor requires nonempty D64 dropout")
        if return_softmax:
            raise ValueError("RNG descriptor does not support diagnostic probabilities")
    if not _rng_state_ok(state, q):
        raise ValueError("rng_state must be a contiguous CUDA int64 tensor of shape [2] on q's device")
    if n == 16:
        reserve, generator = args[14], int(args[15])
        values = [int(x) for x in reserve(generator, q.device.index or 0, q.shape[0] * q.shape[2] * 32)]
        if len(values) != 4 or values[3] not in (0, 1):
            raise ValueError("invalid reserved RNG descriptor")
        descriptor, captured = values[:3], values[3]
        what = "invalid reserved capture pointers"
    else:
        descriptor, captured = [int(x) for x in args[14:17]], int(bool(args[17]))
        what = "invalid capture descriptor pointers"
    if captured and (descriptor[0] == 0 or descriptor[1] == 0 or descriptor[0] % 8 or descriptor[1] % 8):
        raise ValueError(what)
    _resolve_descriptor(state, descriptor, captured)


def _fwd_impl(args, lse_only):
    n = len(args)
    if n not in (9, 10, 12, 13, 14, 16, 18):
        raise ValueError(
            "fwd expects 9 positional arguments (q, k, v, alibi_slopes, softmax_scale, "
            "is_causal, window_size_left, window_size_right, softcap), optionally followed by "
            f"p_dropout, seed, offset, and/or an output tensor; got {n}"
        )
    q, k, v, alibi, scale, causal, wl, wr, softcap = args[:9]
    p, seed, offset, state = 0.0, 0, 0, None
    if n >= 12:
        p = _dropout_p(args[9])
        if isinstance(args[10], torch.Tensor):
            state = args[10]
        else:
            seed = int(args[10])
        offset = int(args[11])
    if offset != 0 and state is not None:
        raise ValueError("offset must be zero when seed is an RNG-state tensor")
    return_softmax = n in (14, 16, 18) and bool(args[13])
    supplied = args[12] if n in (14, 16, 18) else args[-1] if n in (10, 13) else None
    if lse_only and supplied is None:
        raise ValueError("LSE-only forward requires a supplied output")
    if lse_only and return_softmax:
        raise ValueError("LSE-only forward cannot return diagnostic probabilities")
    if return_softmax and (float(np.float32(p)) == 0.0 or state is None):
        raise ValueError("return_softmax requires nonzero dropout and a CUDA RNG-state tensor")
    if q.ndim != 4:
        raise ValueError(f"q must have 4 dimensions [B, S, H, D], got shape {list(q.shape)}")
    if n in (16, 18):
        _fwd_descriptor(args, n, q, k, p, state, return_softmax)
    b, sq, h, d = q.shape
    # Misaligned or strided inputs and an output that the kernels cannot write
    # in place are staged through packed copies inside the C ABI
    # (host/layout.rs:46-125, host/forward/mod.rs:349-376).
    out = supplied if supplied is not None else torch.empty(q.shape, dtype=q.dtype, device=q.device)
    lse = torch.empty((b, h, sq), dtype=torch.float32, device=q.device)
    has_scale, sc = _scale_args(scale)
    descs = [describe(t) for t in (q, k, v, alibi)]
    keep_alive, drop = dropout_arg(p, seed, offset, state)
    scalars = (has_scale, sc, int(bool(causal)), ctypes.c_int64(int(wl)), ctypes.c_int64(int(wr)),
               ctypes.c_double(float(softcap)), drop)
    if return_softmax:
        sk = k.shape[1]
        probabilities = torch.empty((b, h, _round128(sq), _round128(sk)), dtype=q.dtype, device=q.device)
        call("kcr_flash_fwd_softmax", *(ref(x) for x in descs), *scalars, ref(describe(out)),
             ref(describe(lse)), ref(describe(probabilities)), stream_of(q))
        return [out, lse, probabilities]
    call("kcr_flash_fwd", *(ref(x) for x in descs), *scalars, ref(describe(out)), ref(describe(lse)),
         stream_of(q))
    if lse_only:
        return lse
    if n in (14, 16, 18):
        return [out, lse, torch.empty(0, dtype=q.dtype, device=q.device)]
    return [out, lse]


def fwd(*args):
    return _fwd_impl(args, False)


def fwd_lse(*args):
    return _fwd_impl(args, True)


def varlen_fwd_explicit(q, k, v, cu_seqlens_q, cu_seqlens_k, seqused_k, leftpad_k, alibi, scale,
                        causal, left, right, softcap, p, state, max_q, max_k, return_softmax,
                        zero_tensors, block_table=None):
    if block_table is not None:
        return _paged_varlen_fwd(q, k, v, cu_seqlens_q, cu_seqlens_k, seqused_k, leftpad_k, alibi, scale,
                                 causal, left, right, softcap, p, max_q, return_softmax, block_table)
    # host/varlen/mod.rs:201-229
    p = float(p)
    if (not (p == p) or not 0.0 <= p < 1.0 or float(np.float32(p)) >= 1.0
            or (float(np.float32(p)) > 0.0 and float(softcap) > 0.0)
            or (return_softmax and float(np.float32(p)) == 0.0)):
        raise ValueError("invalid dropout, softcap, or probability request")
    if float(np.float32(p)) > 0.0:
        if state is None:
            raise ValueError("dropout requires RNG state")
        if not _rng_state_ok(state, q):
            raise ValueError("RNG state must be contiguous int64 [2] on q's device")
    batch = cu_seqlens_q.numel() - 1
    tq, h, d = q.shape
    hk = k.shape[1]
    if (int(max_q) == 1 and tq == batch and h > hk and hk > 0 and h % hk == 0 and alibi is None
            and float(np.float32(p)) == 0.0 and int(left) < 0 and int(right) < 0):
        return _grouped_decode(q, k, v, cu_seqlens_k, seqused_k, leftpad_k, scale, softcap, max_k,
                               zero_tensors)
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    lse = torch.empty((q.shape[1], q.shape[0]), dtype=torch.float32, device=q.device)
    has_scale, sc = _scale_args(scale)
    descs = [describe(t) for t in (q, k, v, cu_seqlens_q, cu_seqlens_k, seqused_k, leftpad_k, alibi)]
    keep_alive, drop = dropout_arg(p, 0, 0, state)
    scalars = (has_scale, sc, int(bool(causal)), ctypes.c_int64(int(left)), ctypes.c_int64(int(right)),
               ctypes.c_double(float(softcap)), drop, ctypes.c_int64(int(max_q)), ctypes.c_int64(int(max_k)),
               int(bool(zero_tensors)))
    if return_softmax:
        probabilities = torch.empty((batch, h, _round128(max_q), _round128(max_k)), dtype=q.dtype,
                                    device=q.device)
        call("kcr_flash_varlen_fwd_softmax", *(ref(x) for x in descs), *scalars, ref(describe(out)),
             ref(describe(lse)), ref(describe(probabilities)), stream_of(q))
    else:
        probabilities = torch.empty(0, dtype=q.dtype, device=q.device)
        call("kcr_flash_varlen_fwd", *(ref(x) for x in descs), *scalars, ref(describe(out)),
             ref(describe(lse)), stream_of(q))
    return [out, lse, probabilities]


def _grouped_decode(q, k, v, cu_seqlens_k, seqused_k, leftpad_k, scale, softcap, max_k, zero_tensors):
    """One query per sequence with GQA (host/varlen/mod.rs:310-372, packed_grouped):
    the H / Hk query heads of a KV head become the query rows of one sequence, so
    each K/V tile is read once per KV head. A single query sees every key, causal
    or not (varlen/mod.rs:250-268). Returns [out [B, H, D], lse [H, B], probs]."""
    b, h, d = q.shape
    hk = k.shape[1]
    g = h // hk
    qg = q.reshape(b, hk, g, d).transpose(1, 2).reshape(b * g, hk, d).contiguous()
    cu_q = torch.arange(0, (b + 1) * g, g, dtype=torch.int32, device=q.device)
    out_g = torch.empty_like(qg)
    lse_g = torch.empty((hk, b * g), dtype=torch.float32, device=q.device)
    has_scale, sc = _scale_args(scale)
    call("kcr_flash_varlen_fwd", *(ref(describe(t)) for t in (
             qg, k, v, cu_q, cu_seqlens_k, seqused_k, leftpad_k, None)),
         has_scale, sc, 0, ctypes.c_int64(-1), ctypes.c_int64(-1), ctypes.c_double(float(softcap)), None,
         ctypes.c_int64(g), ctypes.c_int64(int(max_k)), int(bool(zero_tensors)), ref(describe(out_g)),
         ref(describe(lse_g)), stream_of(q))
    out = out_g.reshape(b, g, hk, d).transpose(1, 2).reshape(b, h, d)
    lse = lse_g.reshape(hk, b, g).permute(0, 2, 1).reshape(h, b)
    return [out, lse, torch.empty(0, dtype=q.dtype, device=q.device)]


def _paged_varlen_fwd(q, k, v, cu_seqlens_q, cu_seqlens_k, seqused_k, leftpad_k, alibi, scale, causal,
                      left, right, softcap, p, max_q, return_softmax, block_table):
    """varlen_fwd_explicit with a block table (host/varlen/mod.rs:36-54, arg 19):
    k/v are pages [num_pages, page_size, Hk, D]; sequence b reads its first
    seqused_k[b] (or cu_seqlens_k[b + 1] - cu_seqlens_k[b]) keys through
    block_table[b, :]."""
    if float(np.float32(float(p))) > 0.0 or return_softmax:
        raise ValueError("paged K/V does not support dropout or returned probabilities")
    if leftpad_k is not None:
        raise ValueError("paged caches require page size divisible by 256 and no leftpad or cache_batch_idx")
    if seqused_k is None:
        seqused_k = (cu_seqlens_k[1:] - cu_seqlens_k[:-1]).to(torch.int32).contiguous()
    qp = _packed(q)
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    lse = torch.empty((q.shape[1], q.shape[0]), dtype=torch.float32, device=q.device)
    has_scale, sc = _scale_args(scale)
    call("kcr_flash_fwd_kvcache", *(ref(describe(t)) for t in (qp, k, v, cu_seqlens_q, seqused_k)),
         ctypes.c_int64(0), *(ref(describe(t)) for t in (None, None, block_table, alibi)),
         has_scale, sc, int(bool(causal)), ctypes.c_int64(int(left)), ctypes.c_int64(int(right)),
         ctypes.c_double(float(softcap)), ctypes.c_int64(int(max_q)), ctypes.c_int64(1),
         ctypes.c_void_p(0), ctypes.c_int64(0), ref(describe(out)), ref(describe(lse)), stream_of(q))
    return [out, lse, torch.empty(0, dtype=q.dtype, device=q.device)]


def bwd_preprocess(dout, out, p):
    p = float(p)
    if not (p == p) or not 0.0 <= p < 1.0 or float(np.float32(p)) >= 1.0:
        raise ValueError("p_dropout must be in [0, 1) as float32")
    if out.ndim != 4 or dout.shape != out.shape:
        raise ValueError("dout and out must share shape, dtype and device")
    b, s, h, d = out.shape
    rounded = (s + 127) // 128 * 128
    delta = torch.empty((b, h, rounded), dtype=torch.float32, device=out.device)
    call("kcr_flash_bwd_preprocess", ref(describe(dout)), ref(describe(out)),
         ctypes.c_double(float(p)), ref(describe(delta)), stream_of(out))
    return delta


def _bwd(args, want_q, want_kv):
    if len(args) != 14:
        raise ValueError(
            "backward component expects q, k, v, dout, lse, delta, alibi, scale, causal, left, "
            "right, softcap, dropout, rng_state"
        )
    q, k, v, dout, lse, delta, alibi, scale, causal, left, right, softcap, p, rng = args
    p = float(p)
    # host/backward.rs:75-113
    if (not (p == p) or not 0.0 <= p < 1.0 or float(np.float32(p)) >= 1.0
            or (float(np.float32(p)) > 0.0 and float(softcap) > 0.0)):
        raise ValueError("invalid dropout or dropout combined with softcap")
    if float(np.float32(p)) > 0.0:
        if rng is None:
            raise ValueError("dropout backward requires saved RNG state")
        if not _rng_state_ok(rng, q):
            raise ValueError("RNG state must be contiguous CUDA int64 [2] on q's device")
    qp, kp, vp, dp = q, k, v, dout
    dq = torch.empty(q.shape, dtype=q.dtype, device=q.device) if want_q else None
    dk = torch.empty(k.shape, dtype=k.dtype, device=k.device) if want_kv else None
    dv = torch.empty(v.shape, dtype=v.dtype, device=v.device) if want_kv else None
    b, sq, h, d = q.shape
    ws_bytes = lib.kcr_flash_bwd_workspace_bytes(b, h, sq, d)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=q.device)
    has_scale, sc = _scale_args(scale)
    descs = [describe(t) for t in (qp, kp, vp, dp, lse, delta, alibi)]
    keep_alive, drop = dropout_arg(p, 0, 0, rng)
    call("kcr_flash_bwd", *(ref(x) for x in descs), has_scale, sc, int(bool(causal)),
         ctypes.c_int64(int(left)), ctypes.c_int64(int(right)), ctypes.c_double(float(softcap)), drop,
         ref(describe(dq)), ref(describe(dk)), ref(describe(dv)),
         ctypes.c_void_p(ws.data_ptr()), ctypes.c_int64(ws.numel()), stream_of(q))
    return dq, dk, dv


def bwd_dq(*args):
    return _bwd(args, True, False)[0]


def bwd_dkv(*args):
    _, dk, dv = _bwd(args, False, True)
    return [dk, dv]


def bwd_all(*args):
    return list(_bwd(args, True, True))


def varlen_bwd_explicit(q, k, v, dout, out, lse, cu_seqlens_q, cu_seqlens_k, alibi, scale, causal,
                        left, right, softcap, p, state, max_q, max_k, zero_tensors):
    p = float(p)
    if (not (p == p) or not 0.0 <= p < 1.0 or float(np.float32(p)) >= 1.0
            or (float(np.float32(p)) > 0.0 and float(softcap) > 0.0)):
        raise ValueError("invalid dropout or dropout combined with softcap")
    if float(np.float32(p)) > 0.0:
        if state is None:
            raise ValueError("dropout backward requires saved RNG state")
        if not _rng_state_ok(state, q):
            raise ValueError("RNG state must be contiguous CUDA int64 [2] on q's device")
    qp, kp, vp, dp, op = q, k, v, dout, out
    batch = cu_seqlens_q.numel() - 1
    tq, h, d = q.shape
    dq = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    dk = torch.empty(k.shape, dtype=k.dtype, device=k.device)
    dv = torch.empty(v.shape, dtype=v.dtype, device=v.device)
    delta = torch.empty((h, tq + 128 * batch), dtype=torch.float32, device=q.device)
    ws_bytes = lib.kcr_flash_varlen_bwd_workspace_bytes(tq, h, batch, d)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=q.device)
    has_scale, sc = _scale_args(scale)
    descs = [describe(t) for t in (qp, kp, vp, dp, op, lse, cu_seqlens_q, cu_seqlens_k, alibi)]
    keep_alive, drop = dropout_arg(p, 0, 0, state)
    call("kcr_flash_varlen_bwd", *(ref(x) for x in descs), has_scale, sc, int(bool(causal)),
         ctypes.c_int64(int(left)), ctypes.c_int64(int(right)), ctypes.c_double(float(softcap)), drop,
         ctypes.c_int64(int(max_q)), ctypes.c_int64(int(max_k)), int(bool(zero_tensors)),
         ref(describe(dq)), ref(describe(dk)), ref(describe(dv)), ref(describe(delta)),
         ctypes.c_void_p(ws.data_ptr()), ctypes.c_int64(ws.numel()), stream_of(q))
    return [dq, dk, dv, delta]


def _auto_splits(blocks, key_tiles, device):
    """Key splits for an underfilled grid (decode): enough blocks for two per CU,
    at least 4 key tiles per split, at most 128 splits (host/varlen/mod.rs:673)."""
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    if blocks >= 2 * cus or key_tiles < 8:
        return 1
    return int(max(1, min(128, (2 * cus + blocks - 1) // blocks, key_tiles // 4)))


def check_cache_append(q, kcache, k, v, seqlens_k, capacity):
    """flash_attn_interface.py:600-631: the append arguments, checked before
    anything is written."""
    if k is None:
        return
    b, sq = q.shape[0], q.shape[1]
    if seqlens_k is None:
        raise RuntimeError("cache lengths are required when appending K/V")
    for name, t in (("k", k), ("v", v)):
        if (not isinstance(t, torch.Tensor) or t.ndim != 4 or t.shape[0] != b
                or t.shape[2:] != kcache.shape[2:] or t.dtype != q.dtype or t.device != q.device
                or t.stride(-1) != 1):
            raise RuntimeError(
                f"{name} must match query batch and cache heads/dtype/device with unit last stride")
    if k.shape != v.shape or k.shape[1] > capacity or sq > capacity:
        raise RuntimeError("new K/V shapes must match and fit the cache capacity")


def fwd_kvcache(q, kcache, vcache, k=None, v=None, seqlens_k=None, rotary_cos=None, rotary_sin=None,
                cache_batch_idx=None, leftpad_k=None, block_table=None, alibi_slopes=None, out=None,
                softmax_scale=None, is_causal=False, window_size_left=-1, window_size_right=-1,
                softcap=0.0, is_rotary_interleaved=False, num_splits=1, _caches_out=None):
    """Cached inference (flash_attn_interface.py:1474-1700): appends new K/V at
    positions seqlens_k[b] .. (rotating K, and Q, when rotary tables are given),
    then attends over cache rows [leftpad_k[b], seqlens_k[b] + new). Returns
    [out [B, Sq, H, D], lse [B, H, Sq]]. Decode steps (Sq = 1) with GQA treat the
    query heads of a KV head as query rows, as the reference does."""
    for name, t in (("q", q), ("kcache", kcache), ("vcache", vcache)):
        if not isinstance(t, torch.Tensor) or t.ndim != 4:
            raise RuntimeError(f"{name} must be rank 4")
    b, sq, h, d = q.shape
    if not 0 < d <= 256:
        raise RuntimeError("head size must be in 1..256")
    if kcache.shape != vcache.shape or kcache.shape[-1] != d:
        raise RuntimeError("K/V cache shapes must match Q's head size")
    if any(t.stride(-1) != 1 for t in (q, kcache, vcache)):
        raise RuntimeError("Input tensor must have contiguous last dimension")
    splits = int(num_splits)
    if not splits <= 128:
        raise RuntimeError("num_splits must fit int32 and be at most 128")
    left, right = int(window_size_left), int(window_size_right)
    hk = kcache.shape[2]
    if block_table is not None:
        if block_table.ndim != 2 or block_table.shape[0] != b or block_table.dtype != torch.int32:
            raise RuntimeError("block_table must be int32 [batch, max_blocks] with unit last stride on Q's device")
        if kcache.shape[1] % 256 or leftpad_k is not None or cache_batch_idx is not None:
            raise RuntimeError("paged caches require page size divisible by 256 and no leftpad or cache_batch_idx")
        capacity = kcache.shape[1] * block_table.shape[1]
    else:
        capacity = kcache.shape[1]
        if cache_batch_idx is None and kcache.shape[0] < b:
            raise RuntimeError("cache batch is too small for Q")
    if cache_batch_idx is not None and cache_batch_idx.shape != (b,):
        cache_batch_idx = cache_batch_idx.reshape(-1)[:b]
    if k is None and v is not None and not isinstance(v, torch.Tensor):
        raise RuntimeError("v must be a Tensor or None")
    if k is not None and v is None:
        raise RuntimeError("new V is required when new K is supplied")
    if rotary_cos is None:
        # The reference ignores a sine table supplied without a cosine table.
        if rotary_sin is not None and not isinstance(rotary_sin, torch.Tensor):
            raise RuntimeError("rotary_sin must be a Tensor or None")
        rotary_sin = None
    elif rotary_sin is None:
        raise RuntimeError("rotary sin is required when rotary cos is supplied")
    if rotary_cos is not None and k is None:
        raise RuntimeError("rotary tables require new K/V")
    check_cache_append(q, kcache, k, v, seqlens_k, capacity)
    new_keys = 0 if k is None else k.shape[1]
    if d % 8:
        # Head sizes that are not a multiple of 8 run on zero-padded copies; the
        # appended rows are copied back into the caller's caches afterwards
        # (flash_attn_interface.py:1562-1566, 1640-1642).
        pd = (d + 7) // 8 * 8
        pad = (lambda t: None if t is None else torch.nn.functional.pad(t, (0, pd - d)))
        result = fwd_kvcache(pad(q), pad(kcache), pad(vcache), pad(k), pad(v), seqlens_k, rotary_cos,
                             rotary_sin, cache_batch_idx, leftpad_k, block_table, alibi_slopes, None,
                             1.0 / math.sqrt(d) if softmax_scale is None else softmax_scale, is_causal,
                             window_size_left, window_size_right, softcap, is_rotary_interleaved,
                             num_splits, _caches_out=(kcache, vcache) if new_keys > 0 else None)
        output, lse = result
        output = output[..., :d]
        if out is not None:
            out.copy_(output)
            output = out
        return [output, lse]
    causal = bool(is_causal)
    if new_keys > 0:
        rotated = torch.empty_like(q) if rotary_cos is not None else None
        advance_q = causal or 0 <= left < capacity or 0 <= right < capacity
        call("kcr_flash_cache_update", *(ref(describe(t)) for t in (
                 q, kcache, vcache, k, v, seqlens_k, rotary_cos, rotary_sin, cache_batch_idx, block_table)),
             int(bool(is_rotary_interleaved)), int(advance_q), ref(describe(rotated)), stream_of(q))
        if rotated is not None:
            q = rotated
        if _caches_out is not None:
            # Padded copies: write the appended rows back to the caller's caches.
            _caches_out[0].copy_(kcache[..., :_caches_out[0].shape[-1]])
            _caches_out[1].copy_(vcache[..., :_caches_out[1].shape[-1]])
        else:
            # Native writes bypass torch's in-place ops: bump the versions so
            # autograd sees the caches changed.
            torch.autograd.graph.increment_version((kcache, vcache))
    # Cache rows attended: [leftpad, seqlens_k + new) (all rows without lengths);
    # the kernels add new_keys to the lengths.
    used = None if seqlens_k is None else seqlens_k.to(torch.int32).contiguous()
    grouped = sq == 1 and h > hk and left < 0 and right < 0 and alibi_slopes is None
    # The kernels take q / out as [B, rows, heads, D] views and lse as [B, heads, rows]
    # through their strides, so the caller's tensors are used in place.
    if out is not None and out.shape != q.shape and not (grouped and tuple(out.shape) == (b, h // hk, hk, d)):
        raise RuntimeError("out must match Q or its grouped layout and have unit last stride")
    if out is not None and out.stride(-1) != 1:
        raise RuntimeError("out must match Q or its grouped layout and have unit last stride")
    output = out if out is not None else torch.empty_like(q, memory_format=torch.contiguous_format)
    lse = torch.empty((b, h, sq), dtype=torch.float32, device=q.device)
    if grouped:
        # Query heads hk * G .. hk * G + G - 1 become the G query rows of KV head hk
        # (host/varlen/mod.rs:310-372); one query row sees every key either way.
        g = h // hk
        rows, heads = g, hk
        causal = False
        qp = q.reshape(b, hk, g, d).transpose(1, 2)
        if tuple(output.shape) == (b, g, hk, d):
            # The grouped decode layout [B, H / Hk, Hk, D] (flash_attn_interface.py:672-700,
            # 1647-1651) is already [B, rows, heads, D].
            op = output
        else:
            op = output.view(b, hk, g, d).transpose(1, 2) if output.is_contiguous() else None
        lse_p = lse.view(b, hk, g)
    else:
        rows, heads = sq, h
        qp, op, lse_p = q, output, lse
    if not _rows_aligned(qp):
        qp = qp.contiguous()
    # The attention kernels move 16-byte row chunks: caches with unaligned rows
    # are read through an aligned copy (host/layout.rs:46-125).
    kc_att = kcache if _rows_aligned(kcache) else kcache.contiguous()
    vc_att = vcache if _rows_aligned(vcache) else vcache.contiguous()
    tmp = op is None or not _rows_aligned(op)
    if tmp:
        op = torch.empty((b, rows, heads, d), dtype=q.dtype, device=q.device)
    if splits < 1:
        splits = _auto_splits(b * heads * ((rows + 127) // 128), (capacity + 63) // 64, q.device)
    ws_bytes = lib.kcr_flash_fwd_kvcache_workspace_bytes(splits, heads, b * rows, d)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=q.device)
    has_scale, sc = _scale_args(softmax_scale)
    call("kcr_flash_fwd_kvcache", *(ref(describe(t)) for t in (qp, kc_att, vc_att, None, used)),
         ctypes.c_int64(0 if used is None else new_keys),
         *(ref(describe(t)) for t in (leftpad_k, cache_batch_idx, block_table, alibi_slopes)),
         has_scale, sc, int(causal), ctypes.c_int64(left), ctypes.c_int64(right),
         ctypes.c_double(float(softcap)), ctypes.c_int64(rows), ctypes.c_int64(splits),
         ctypes.c_void_p(ws.data_ptr()), ctypes.c_int64(ws.numel()), ref(describe(op)),
         ref(describe(lse_p)), stream_of(q))
    if tmp:
        if tuple(output.shape) == tuple(op.shape):
            output.copy_(op)
        else:
            output.copy_(op.transpose(1, 2).reshape(b, 1, h, d))
    if tuple(output.shape) != (b, sq, h, d):
        # Grouped layout out: returned in head order as [B, 1, H, D].
        output = output.transpose(1, 2).reshape(b, 1, h, d)
    return [output, lse]


ops = SimpleNamespace(
    rng_state=rng_state,
    fwd=fwd,
    fwd_lse=fwd_lse,
    varlen_fwd_explicit=varlen_fwd_explicit,
    bwd_preprocess=bwd_preprocess,
    bwd_dq=bwd_dq,
    bwd_dkv=bwd_dkv,
    bwd_all=bwd_all,
    varlen_bwd_explicit=varlen_bwd_explicit,
    fwd_kvcache=fwd_kvcache,
)
