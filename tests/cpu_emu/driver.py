"""Drives the library's C ABI on the CPU executor (test infrastructure).

``Emu(asan)`` loads ``_build/libsgd_emu[_asan].so`` (see build.py; the ASan build needs
clang's ASan runtime preloaded, which ``run_case.py`` arranges in a child process).
Device buffers are host allocations of exactly the size a device buffer would have,
filled with garbage like fresh device memory, so AddressSanitizer sees every access
past a buffer's end.  ``decode()`` makes the calls DecodeEngine.prepare()/execute()
make -- the fused plan build with the layer's counters, the attention launch (writing
single-split rows to the output) and the split merge of the other rows -- with the same
argument marshalling.
"""
import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (os.path.join(ROOT, "-sglang-decode-_amd"), ROOT, HERE):
    if p not in sys.path:
        sys.path.insert(0, p)

from sglang_decode import _lib  # noqa: E402  (ctypes structs and signatures only)

import build as B  # noqa: E402


class Emu:
    def __init__(self, asan=False, cus=256):
        self.lib = ctypes.CDLL(B.lib_path(asan))
        for name, (res, args) in _lib._SIGNATURES.items():
            fn = getattr(self.lib, name, None)
            if fn is not None:
                fn.restype, fn.argtypes = res, args
        self.lib.emu_alloc.restype = ctypes.c_void_p
        self.lib.emu_alloc.argtypes = [ctypes.c_size_t]
        self.lib.emu_free.argtypes = [ctypes.c_void_p]
        self.lib.emu_set_cus.argtypes = [ctypes.c_int]
        self.lib.emu_set_cus(cus)
        self._held = []

    def array(self, shape, dtype, fill=None):
        """A 'device' array: host memory of exactly the buffer's size (garbage unless filled)."""
        shape = tuple(int(s) for s in np.atleast_1d(shape)) if not isinstance(shape, tuple) else shape
        dtype = np.dtype(dtype)
        nbytes = int(np.prod(shape, dtype=np.int64)) * dtype.itemsize
        p = self.lib.emu_alloc(nbytes)
        self._held.append(p)
        raw = (ctypes.c_uint8 * max(nbytes, 1)).from_address(p)
        a = np.frombuffer(raw, dtype=np.uint8, count=nbytes).view(dtype).reshape(shape)
        if fill is not None:
            a[...] = fill
        return a

    def upload(self, x, dtype=None):
        x = np.ascontiguousarray(x if dtype is None else np.asarray(x, dtype=dtype))
        a = self.array(x.shape, x.dtype)
        a[...] = x
        return a

    def check(self, rc, what):
        if rc != 0:
            msg = self.lib.sgd_last_error().decode(errors="replace")
            raise (ValueError if rc == _lib.SGD_EINVAL else RuntimeError)(f"{what}: {msg}")


def ptr(a):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def bits16(t):
    """torch bf16/fp16 tensor -> uint16 numpy array of its bits."""
    import torch
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits16(a, dtype_code):
    a = np.asarray(a, dtype=np.uint16)
    if dtype_code == _lib.SGD_BF16:
        return (a.astype(np.uint32) << 16).view(np.float32)
    return a.view(np.float16).astype(np.float32)


class Plan:
    """PlanBuffers of the executor: same fields, shapes and zero initialization."""

    def __init__(self, emu, config, rules=()):
        self.config = c = config
        b, e, t = c.batch_capacity, c.record_capacity, c.task_capacity
        z = lambda n: emu.array((n,), np.int32, 0)
        self.lengths, self.splits, self.active = z(b), z(b), z(1)
        self.counts, self.offsets, self.chunk = z(b), z(b + 1), z(b)
        self.request, self.split, self.begin, self.end, self.weight = [z(e) for _ in range(5)]
        self.order, self.pack_first, self.pack_count = z(e), z(t), z(t)
        self.record_count, self.num_packs, self.mode, self.error = [z(1) for _ in range(4)]
        self.static_head, self.static_next = z(c.workers), z(t)
        self.dispatch = emu.array((t, 8), np.int32, 0)
        rows = [[r.min_tasks, r.max_tasks, r.min_ratio, r.max_ratio, r.mode] for r in rules]
        self.rules = emu.upload(np.array(rows or [[0, 0, 100, 100, 1]], dtype=np.int32))
        self.rule_count = len(rows)

    def c_struct(self):
        c, s = self.config, _lib.PlanBuffersC()
        for name in ("lengths", "splits", "active", "counts", "offsets", "chunk", "request", "split", "begin",
                     "end", "weight", "order", "pack_first", "pack_count", "record_count", "num_packs", "mode",
                     "error", "static_head", "static_next", "rules", "dispatch"):
            setattr(s, name, getattr(self, name).ctypes.data)
        s.rule_count = self.rule_count
        s.batch_capacity, s.max_splits, s.max_context = c.batch_capacity, c.max_splits, c.max_context
        s.kv_heads, s.workers, s.block_kv, s.buckets = c.kv_heads, c.workers, c.block_kv, c.buckets
        return s

    def read(self):
        g = lambda a: a.tolist()
        d = {k: g(getattr(self, k)) for k in ("counts", "offsets", "chunk", "request", "split", "begin", "end",
                                               "weight", "order", "pack_first", "pack_count", "static_head",
                                               "static_next")}
        d.update({k: int(getattr(self, k)[0]) for k in ("record_count", "num_packs", "mode", "error")})
        return d


def decode(emu, config, lengths, splits, q, k, v, pages, indptr=None, *, mode=-1, kernel="auto", scale=None,
           rules=(), run_greedy=None, poison=True, direct=True):
    """One prepare() + execute() on the executor.  q/k/v: torch CPU tensors (bf16/fp16);
    pages: paged table [Bcap, max_pages] or CSR kv_indices; indptr: CSR kv_indptr or None.
    Returns dict(out [Bcap,Hq,D] float32, partial, lse, plan, kernel)."""
    import torch
    c = config
    dt = _lib.dtype_code(q.dtype)
    plan = Plan(emu, c, rules)
    n = len(lengths)
    plan.lengths[:n] = lengths
    plan.splits[:] = 1
    plan.splits[:n] = splits
    plan.active[0] = n
    sync = emu.array((2,), np.int32, 0)
    shape = (c.batch_capacity, c.query_heads, c.max_splits)
    partial = emu.array((*shape, c.head_dim), np.float32, np.nan if poison else None)
    lse = emu.array(shape, np.float32, np.nan if poison else None)
    out = emu.array((c.batch_capacity, c.query_heads, c.head_dim), np.uint16, 0x7fc0 if poison else None)
    if run_greedy is None:
        run_greedy = int(mode) == 2 or any(int(r.mode) == 2 for r in rules)
    emu.check(emu.lib.sgd_build_plan(ctypes.byref(plan.c_struct()), int(mode), int(bool(run_greedy)),
                                     ptr(sync), 2, None), "build_plan")
    qd, kd, vd = emu.upload(bits16(q)), emu.upload(bits16(k)), emu.upload(bits16(v))
    pd = emu.upload(pages.detach().cpu().numpy().astype(np.int32))
    ipd = emu.upload(indptr.detach().cpu().numpy().astype(np.int32)) if indptr is not None else None
    a = _lib.DecodeArgsC()
    a.q, a.k, a.v, a.pages = qd.ctypes.data, kd.ctypes.data, vd.ctypes.data, pd.ctypes.data
    a.indptr = ipd.ctypes.data if ipd is not None else None
    for name in ("lengths", "request", "split", "begin", "end", "order", "offsets", "chunk", "active",
                 "record_count", "mode", "pack_first", "pack_count", "num_packs", "static_head", "static_next"):
        setattr(a, name, getattr(plan, name).ctypes.data)
    a.counter, a.done_counter = sync.ctypes.data, sync[1:].ctypes.data
    a.partial, a.lse = partial.ctypes.data, lse.ctypes.data
    a.dispatch, a.dispatch_units = plan.dispatch.ctypes.data, plan.dispatch.shape[0]
    a.scale = float(c.head_dim ** -0.5 if scale is None else scale)
    a.q_stride[:] = list(q.stride())
    if indptr is None:
        a.k_stride[:], a.v_stride[:], a.pt_stride[:] = list(k.stride()), list(v.stride()), list(pages.stride())
        a.csr = 0
    else:
        a.k_stride[:] = [k.stride(0), 0, k.stride(1), k.stride(2)]
        a.v_stride[:] = [v.stride(0), 0, v.stride(1), v.stride(2)]
        a.pt_stride[:] = [0, 0]
        a.csr = 1
    a.query_heads, a.kv_heads, a.head_dim = c.query_heads, c.kv_heads, c.head_dim
    a.max_splits, a.page_size, a.dtype, a.workers = c.max_splits, c.page_size, dt, c.workers
    a.kernel = _lib.KERNELS[kernel]
    if direct:  # single-split rows straight from the attention, as DecodeEngine.execute does
        a.out = out.ctypes.data
    emu.check(emu.lib.sgd_persistent_decode(ctypes.byref(a), None), "persistent_decode")
    ran = _lib.KERNEL_NAMES[emu.lib.sgd_attention_kernel(ctypes.byref(a))]
    emu.check(emu.lib.sgd_merge_splits_min(
        ptr(partial), ptr(lse), ptr(plan.counts), ptr(plan.active), ptr(plan.error), ptr(out),
        c.batch_capacity, c.query_heads, c.head_dim, c.max_splits, 2 if direct else 1, dt, None), "merge_splits")
    return dict(out=from_bits16(out, dt).reshape(out.shape), partial=np.array(partial), lse=np.array(lse),
                plan=plan.read(), kernel=ran, sync=sync.tolist())
