"""Persistent decode attention launch (kernel in csrc/attention*.hip).

``persistent_decode`` marshals one launch the way runtime/engine.py:63-70 of the
reference does, but passes element strides as runtime int64 arguments instead
of compile-time constants, so a new layout never recompiles anything.
"""
import ctypes

from .. import _lib
from .._lib import DecodeArgsC, check, ptr


def persistent_decode(plan, layer, q, k, v, pages, indptr, scale, k_strides, v_strides,
                      pt_strides, csr, kernel="auto"):
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
    check(_lib.lib().sgd_persistent_decode(ctypes.byref(a), _lib.stream_handle(q.device)),
          "persistent_decode")
    return _lib.KERNEL_NAMES[_lib.lib().sgd_attention_kernel(ctypes.byref(a))]
