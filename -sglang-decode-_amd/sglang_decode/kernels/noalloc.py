"""One decode step with no device allocation (csrc/noalloc.hip, ``sgd_decode_noalloc``).

For callers that cannot allocate device memory -- code under HIP graph capture, tight
serving loops: the plan tables, claim counters and split partial/LSE slots live in a
32 MiB array the library holds on each GPU, so only the inputs and ``out`` are passed.
Same launches and results as DecodeEngine's prepare() + execute() with no policy
rules.  Calls that overlap on one GPU race on the array.
"""
import ctypes

import torch

from .. import _lib
from .._lib import NoAllocArgsC, check
from .attention import checked_layout


def decode_noalloc(config, q, k, v, pages, lengths, splits, active, out, *, indptr=None, scale=None,
                   force_mode=-1, kernel="auto"):
    """q [Bcap, Hq, D]; k/v paged [pages, page, Hkv, D] (pages = table [Bcap, max_pages]) or
    CSR [tokens, Hkv, D] (pages = kv_indices, indptr = kv_indptr); lengths / splits int32
    [Bcap] and active int32 [1] on the device; out [Bcap, Hq, D] in q's dtype."""
    c = config
    ks, vs, pts, csr = checked_layout(c, q, k, v, pages, indptr, out.dtype, who="decode_noalloc")
    for name, t, n in (("lengths", lengths, c.batch_capacity), ("splits", splits, c.batch_capacity),
                       ("active", active, 1)):
        # the plan launch reads lengths[r] and splits[r] for every r < Bcap
        if t.dtype != torch.int32 or t.device != q.device or t.numel() != n or not t.is_contiguous():
            raise ValueError(f"decode_noalloc: {name} must be a contiguous int32 tensor of {n} entries on q's device")
    if tuple(out.shape) != (c.batch_capacity, c.query_heads, c.head_dim) or not out.is_contiguous() or \
            out.device != q.device:
        raise ValueError("decode_noalloc: out must be a contiguous [Bcap, Hq, D] tensor of q's dtype on q's device")
    a = NoAllocArgsC()
    a.q, a.k, a.v, a.pages = q.data_ptr(), k.data_ptr(), v.data_ptr(), pages.data_ptr()
    a.indptr = indptr.data_ptr() if indptr is not None else None
    a.lengths, a.splits, a.active, a.out = lengths.data_ptr(), splits.data_ptr(), active.data_ptr(), out.data_ptr()
    a.scale = float(c.head_dim ** -0.5 if scale is None else scale)
    a.q_stride[:] = list(q.stride())
    a.k_stride[:], a.v_stride[:], a.pt_stride[:] = list(ks), list(vs), list(pts)
    a.batch_capacity, a.max_splits, a.max_context = c.batch_capacity, c.max_splits, c.max_context
    a.query_heads, a.kv_heads, a.head_dim = c.query_heads, c.kv_heads, c.head_dim
    a.page_size, a.csr, a.dtype = c.page_size, int(csr), _lib.dtype_code(q.dtype)
    a.workers = c.workers
    a.force_mode = int(force_mode)
    a.kernel = _lib.KERNELS[kernel] if isinstance(kernel, str) else int(kernel)
    check(_lib.lib().sgd_decode_noalloc(ctypes.byref(a), _lib.stream_handle(q.device)), "decode_noalloc")
    return out
