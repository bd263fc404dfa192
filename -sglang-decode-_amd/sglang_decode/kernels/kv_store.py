"""The decode step's KV-pool write and q staging in one launch (kernel in csrc/kv_store.hip).

Replaces, in the reference adapter (integrations/sglang_backend.py:91-92, 102-103),
``token_to_kv_pool.set_kv_buffer(layer, out_cache_loc, k, v)`` -- upstream a scatter of
k and one of v into the layer's pools -- and ``qbuf[:batch].copy_(q.view(batch, Hq, D))``.
"""
import ctypes

import torch

from .. import _lib
from .._lib import check


def _strides2(t, name):
    if t.dim() != 3 or t.stride(2) != 1:
        raise ValueError(f"{name}: expected a [n, heads, head_dim] view with unit last stride, got "
                         f"shape {tuple(t.shape)} strides {t.stride()}")
    return t.stride(0), t.stride(1)


def store_kv_and_stage_q(k_new=None, v_new=None, loc=None, k_cache=None, v_cache=None, q_in=None, q_out=None):
    """k_cache[loc[b]] = k_new[b] and v_cache[loc[b]] = v_new[b] for b < batch (skipped when
    k_new is None), and q_out[b] = q_in[b] (skipped when q_in is None), bit for bit.

    k_new / v_new: [batch, Hkv, D]; k_cache / v_cache: [tokens, Hkv, D]; loc: int32 or int64
    [batch]; q_in: [batch, Hq, D]; q_out: [>= batch, Hq, D].  Every tensor on one device, one
    16-bit dtype, unit last stride, 16-byte aligned rows.  A slot outside [0, tokens) is
    skipped on the device (callers that need torch's index check do it on the host)."""
    if k_new is None and q_in is None:
        return
    ref = k_new if k_new is not None else q_in
    dtype, device = ref.dtype, ref.device
    batch = ref.shape[0]
    args = dict(new=None, loc=None, lbits=0, cache=None, tokens=0, qi=None, qo=None, hkv=1, hq=1)
    head_dim = ref.shape[-1]
    keep = []
    if k_new is not None:
        for name, t in (("v_new", v_new), ("k_cache", k_cache), ("v_cache", v_cache), ("loc", loc)):
            if t is None:
                raise ValueError(f"store_kv_and_stage_q: {name} is required with k_new")
        if v_new.shape != k_new.shape or k_cache.shape != v_cache.shape or k_cache.shape[1:] != k_new.shape[1:]:
            raise ValueError(f"store_kv_and_stage_q: k/v {tuple(k_new.shape)}/{tuple(v_new.shape)} and caches "
                             f"{tuple(k_cache.shape)}/{tuple(v_cache.shape)} disagree")
        if loc.dim() != 1 or loc.shape[0] < batch or loc.dtype not in (torch.int32, torch.int64):
            raise ValueError("store_kv_and_stage_q: loc must be int32/int64 [>= batch]")
        for t in (v_new, k_cache, v_cache, loc):
            if t.device != device:
                raise ValueError("store_kv_and_stage_q: all tensors must be on one device")
        for t in (v_new, k_cache, v_cache):
            if t.dtype != dtype:
                raise ValueError("store_kv_and_stage_q: K/V and caches must share one dtype (no conversion)")
        loc = loc.contiguous()
        keep.append(loc)
        new = (ctypes.c_int64 * 4)(*_strides2(k_new, "k_new"), *_strides2(v_new, "v_new"))
        cache = (ctypes.c_int64 * 4)(*_strides2(k_cache, "k_cache"), *_strides2(v_cache, "v_cache"))
        args.update(new=new, loc=loc, lbits=int(loc.dtype == torch.int64), cache=cache, tokens=k_cache.shape[0],
                    hkv=k_new.shape[1])
    if q_in is not None:
        if q_out is None or q_out.dim() != 3 or q_in.shape[1:] != q_out.shape[1:] or q_out.shape[0] < q_in.shape[0]:
            raise ValueError("store_kv_and_stage_q: q_out must be [>= batch, Hq, D] like q_in")
        if q_in.shape[0] != batch or q_in.shape[-1] != head_dim:
            raise ValueError("store_kv_and_stage_q: q_in and k_new disagree on batch or head_dim")
        if q_in.dtype != dtype or q_out.dtype != dtype or q_in.device != device or q_out.device != device:
            raise ValueError("store_kv_and_stage_q: q_in / q_out must match the K/V dtype and device")
        args.update(qi=(ctypes.c_int64 * 2)(*_strides2(q_in, "q_in")),
                    qo=(ctypes.c_int64 * 2)(*_strides2(q_out, "q_out")), hq=q_in.shape[1])
    p = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None
    check(_lib.lib().sgd_store_kv_stage_q(
        p(k_new), p(v_new), args["new"], p(args["loc"]), args["lbits"], p(k_cache), p(v_cache), args["cache"],
        args["tokens"], p(q_in), args["qi"], p(q_out), args["qo"], batch, args["hkv"], args["hq"], head_dim,
        _lib.dtype_code(dtype), _lib.stream_handle(device)), "store_kv_and_stage_q")
