"""Persistent decode attention launch (kernel in csrc/attention*.hip).

``persistent_decode`` marshals one launch the way runtime/engine.py:63-70 of the
reference does, but passes element strides as runtime int64 arguments instead
of compile-time constants, so a new layout never recompiles anything.
"""
import ctypes

import torch

from .. import _lib
from .._lib import DecodeArgsC, check, ptr


def checked_layout(config, q, k, v, pages, indptr, out_dtype=None, who="execute"):
    """Host checks of one layer's q, K/V and page metadata against ``config`` (ValueError
    before any launch; the kernels read rows and indices through these shapes), returning
    (k strides, v strides, page-table strides, csr) as element strides.

    KV layouts: paged ``[pages, page_size, kv_heads, D]`` with a page table ``[Bcap,
    max_pages]``, or CSR ``[tokens, kv_heads, D]`` with ``pages`` = kv_indices (1-D) and
    ``indptr`` = kv_indptr (page_size 1)."""
    c = config
    if q.dtype not in (torch.float16, torch.bfloat16) or (k.dtype, v.dtype) != (q.dtype, q.dtype):
        raise ValueError(f"{who}: q, k and v must share one 16-bit dtype (bf16 or fp16), got {q.dtype}, "
                         f"{k.dtype}, {v.dtype}")
    if out_dtype is not None and q.dtype != out_dtype:
        raise ValueError(f"{who}: q is {q.dtype} but the output is {out_dtype}")
    if tuple(q.shape) != (c.batch_capacity, c.query_heads, c.head_dim):
        raise ValueError(f"{who}: q must be [{c.batch_capacity}, {c.query_heads}, {c.head_dim}] (the batch "
                         "capacity; rows past the active batch are ignored)")
    if any(t.device != q.device for t in (k, v, pages)):
        raise ValueError(f"{who}: q, k, v and the page table must be on one device")
    if pages.dtype != torch.int32:
        raise ValueError(f"{who}: the page table / kv_indices must be int32")
    if indptr is None:
        want = (c.page_size, c.kv_heads, c.head_dim)
        if k.ndim != 4 or k.shape != v.shape or tuple(k.shape[1:]) != want:
            raise ValueError(f"{who}: paged K and V must both be [pages, {want[0]}, {want[1]}, {want[2]}], got "
                             f"{tuple(k.shape)} and {tuple(v.shape)}")
        if tuple(pages.shape) != (c.batch_capacity, c.max_pages):
            raise ValueError(f"{who}: page table must be [{c.batch_capacity}, {c.max_pages}], got "
                             f"{tuple(pages.shape)}")
        return k.stride(), v.stride(), pages.stride(), False
    if k.ndim != 3 or k.shape != v.shape or tuple(k.shape[1:]) != (c.kv_heads, c.head_dim):
        raise ValueError(f"{who}: CSR K and V must both be [tokens, {c.kv_heads}, {c.head_dim}], got "
                         f"{tuple(k.shape)} and {tuple(v.shape)}")
    if c.page_size != 1 or pages.ndim != 1:
        raise ValueError(f"{who}: the CSR layout needs page_size 1 and a 1-D kv_indices tensor")
    if indptr.dtype != torch.int32 or indptr.device != q.device or indptr.ndim != 1:
        raise ValueError(f"{who}: kv_indptr must be a 1-D int32 tensor on q's device")
    # a token row is [Hkv, D]: the in-page stride does not exist
    return ((k.stride(0), 0, k.stride(1), k.stride(2)), (v.stride(0), 0, v.stride(1), v.stride(2)),
            (0, 0), True)


def persistent_decode(plan, layer, q, k, v, pages, indptr, scale, k_strides, v_strides,
                      pt_strides, csr, kernel="auto", write_single=False):
    """One attention launch.  ``write_single``: the tasks that are their request's only
    split also write their row of ``layer.output`` (contiguous [Bcap, Hq, D] in q's dtype),
    so the merge may skip those rows (kernels.merge.merge_splits with min_splits 2)."""
    c = plan.config
    a = DecodeArgsC()
    a.q, a.k, a.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
    a.pages = pages.data_ptr()
    a.indptr = indptr.data_ptr() if indptr is not None else None
    for name in ("lengths", "request", "split", "begin", "end", "order", "offsets", "chunk",
                 "active", "record_count", "mode", "pack_first", "pack_count", "num_packs",
                 "static_head", "static_next"):
        setattr(a, name, getattr(plan, name).data_ptr())
    a.counter = layer.counter.data_ptr()
    done = getattr(layer, "done", None)
    a.done_counter = done.data_ptr() if done is not None else None
    a.partial = layer.partial.data_ptr()
    a.lse = layer.lse.data_ptr()
    if getattr(plan, "dispatch_valid", False):
        a.dispatch, a.dispatch_units = plan.dispatch.data_ptr(), plan.dispatch.shape[0]
    a.scale = float(scale)
    a.q_stride[:] = list(q.stride())
    a.k_stride[:] = list(k_strides)
    a.v_stride[:] = list(v_strides)
    a.pt_stride[:] = list(pt_strides)
    a.query_heads, a.kv_heads, a.head_dim = c.query_heads, c.kv_heads, c.head_dim
    a.max_splits, a.page_size, a.csr = c.max_splits, c.page_size, int(bool(csr))
    a.dtype = _lib.dtype_code(q.dtype)
    a.workers = c.workers
    a.kernel = _lib.KERNELS[kernel] if isinstance(kernel, str) else int(kernel)
    if write_single:
        a.out = layer.output.data_ptr()
    check(_lib.lib().sgd_persistent_decode(ctypes.byref(a), _lib.stream_handle(q.device)),
          "persistent_decode")
    return _lib.KERNEL_NAMES[_lib.lib().sgd_attention_kernel(ctypes.byref(a))]
