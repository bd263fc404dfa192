"""Upstream SGLang's two-stage split-KV decode on gfx950 (``sgd_upstream_decode``): the
comparator the reference benchmarks the persistent path against (benchmarks/baselines.py:
8-34), with upstream's call signature (third_party/sglang/decode_attention.py,
``decode_attention_fwd``, SGLang v0.4.6.post5).  Comparison only; the persistent engine
does not use it."""
import ctypes

import torch

from .. import _lib
from .._lib import check, ptr


def decode_attention_fwd(q, k_buffer, v_buffer, o, kv_indptr, kv_indices, attn_logits, attn_lse, num_kv_splits,
                         max_kv_splits, sm_scale):
    """q [batch, Hq, D]; k_buffer / v_buffer [tokens, Hkv, D]; o [batch, Hq, D] (contiguous);
    kv_indptr int32 [batch + 1], kv_indices int32, num_kv_splits int32 [batch];
    attn_logits fp32 [batch, Hq, max_kv_splits, D] and attn_lse fp32 [batch, Hq,
    max_kv_splits] (contiguous) receive the split partials and LSEs."""
    if q.ndim != 3 or k_buffer.ndim != 3 or v_buffer.shape != k_buffer.shape:
        raise ValueError("decode_attention_fwd: q must be [batch, Hq, D] and k_buffer / v_buffer one "
                         "[tokens, Hkv, D] shape")
    batch, hq, d = q.shape
    hkv = k_buffer.shape[1]
    if k_buffer.shape[2] != d or (k_buffer.dtype, v_buffer.dtype) != (q.dtype, q.dtype):
        raise ValueError("decode_attention_fwd: k_buffer / v_buffer must match q's head_dim and dtype")
    tensors = (q, k_buffer, v_buffer, o, kv_indptr, kv_indices, attn_logits, attn_lse, num_kv_splits)
    if any(t.device != q.device for t in tensors):
        raise ValueError("decode_attention_fwd: every tensor must be on q's device")
    # both stages read kv_indptr[b + 1] and num_kv_splits[b] for every b < batch
    for name, t, n in (("kv_indptr", kv_indptr, batch + 1), ("kv_indices", kv_indices, 0),
                       ("num_kv_splits", num_kv_splits, batch)):
        if t.dtype != torch.int32 or not t.is_contiguous() or t.numel() < n:
            raise ValueError(f"decode_attention_fwd: {name} must be contiguous int32 with at least {n} entries")
    if (tuple(attn_logits.shape) != (batch, hq, max_kv_splits, d) or tuple(attn_lse.shape) != (batch, hq, max_kv_splits)
            or not (attn_logits.is_contiguous() and attn_lse.is_contiguous())):
        raise ValueError("decode_attention_fwd: attn_logits / attn_lse must be contiguous [batch, Hq, max_kv_splits"
                         "(, D)] fp32")
    if tuple(o.shape) != (batch, hq, d) or not o.is_contiguous() or o.dtype != q.dtype:
        raise ValueError("decode_attention_fwd: o must be a contiguous [batch, Hq, D] tensor of q's dtype")
    if k_buffer.stride(2) != 1 or v_buffer.stride(2) != 1:
        raise ValueError("decode_attention_fwd: K/V need a unit head_dim stride")
    qs = (ctypes.c_int64 * 3)(*q.stride())
    kvs = (ctypes.c_int64 * 4)(k_buffer.stride(0), k_buffer.stride(1), v_buffer.stride(0), v_buffer.stride(1))
    check(_lib.lib().sgd_upstream_decode(
        ptr(q), ptr(k_buffer), ptr(v_buffer), ptr(o), ptr(kv_indptr), ptr(kv_indices), ptr(attn_logits),
        ptr(attn_lse), ptr(num_kv_splits), batch, int(max_kv_splits), hq, hkv, d, qs, kvs, float(sm_scale),
        _lib.dtype_code(q.dtype), _lib.stream_handle(q.device)), "upstream decode_attention_fwd")
    return o
