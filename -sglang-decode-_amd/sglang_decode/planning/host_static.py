"""Host-planned STATIC schedule: the "strong static" baseline of the reference's benchmark.

benchmarks/bench_decode.py:14-30 of the reference plans the STATIC lists on the host
(heap LPT over the records, planning/reference.py:57-67) on every call, builds the R1
plan on the device for the common records, then replaces only the dispatch metadata:
static_head / static_next uploaded, mode forced to STATIC.

Here the LPT runs in C++ (``sgd_host_static_lists``) and writes straight into pinned
host staging buffers, which are uploaded with asynchronous copies on the current
stream.  ``HostStatic`` keeps the uploaded lists in fixed device buffers, so that
installing them over an R1 plan (``apply``) is three device operations a hipGraph can
capture; ``plan_lists`` re-plans when the lengths change, and ``prepare`` is the
reference's per-call boundary (LPT + upload + R1 build + install).
"""
import ctypes

import numpy as np
import torch

from .. import _lib
from ..config import Mode
from .reference import split_records


def host_static_lists(weights, kv_heads, workers, task_capacity, heads=None, nxt=None):
    """(static_head [workers], static_next [task_capacity]) int32 host arrays, -1 terminated.
    ``heads`` / ``nxt``: optional int32 host arrays to write into (e.g. pinned memory)."""
    w = np.ascontiguousarray(np.asarray(weights, dtype=np.int32))
    heads = np.empty(workers, dtype=np.int32) if heads is None else heads
    nxt = np.empty(task_capacity, dtype=np.int32) if nxt is None else nxt
    if heads.shape != (workers,) or nxt.shape != (task_capacity,) or heads.dtype != np.int32 or \
            nxt.dtype != np.int32 or not (heads.flags.c_contiguous and nxt.flags.c_contiguous):
        raise ValueError("host_static_lists: output arrays must be contiguous int32 [workers] / [task_capacity]")
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    _lib.check(_lib.lib().sgd_host_static_lists(p(w), len(w), kv_heads, workers, task_capacity,
                                                p(heads), p(nxt)), "host_static_lists")
    return heads, nxt


class HostStatic:
    """Host LPT lists of one engine's plan: pinned host staging, fixed device copies."""

    def __init__(self, engine):
        self.engine = engine
        p = engine.plan
        self.heads = torch.full_like(p.static_head, -1)
        self.next = torch.full_like(p.static_next, -1)
        pinned = p.device.type == "cuda"
        self._host_heads = torch.empty(p.static_head.shape, dtype=torch.int32, pin_memory=pinned)
        self._host_next = torch.empty(p.static_next.shape, dtype=torch.int32, pin_memory=pinned)
        self._uploaded = torch.cuda.Event() if pinned else None
        self._pending = False

    def plan_lists(self, lengths, splits):
        """Host LPT for these lengths/splits (ValueError beyond the capacities), written to
        the pinned staging buffers and copied to the fixed device buffers asynchronously on
        the current stream.  The staging buffers are reused: a call first waits for the
        previous call's copies to have left them."""
        c = self.engine.config
        records, _, _ = split_records(lengths, splits, c)
        if self._pending:
            self._uploaded.synchronize()
        host_static_lists([r.weight for r in records], c.kv_heads, c.workers, c.task_capacity,
                          self._host_heads.numpy(), self._host_next.numpy())
        self.heads.copy_(self._host_heads, non_blocking=True)
        self.next.copy_(self._host_next, non_blocking=True)
        if self._uploaded is not None:
            self._uploaded.record()
            self._pending = True

    def apply(self):
        """After an R1 ``prepare()``: install the lists and force STATIC (device ops only)."""
        p = self.engine.plan
        p.static_head.copy_(self.heads)
        p.static_next.copy_(self.next)
        p.mode.fill_(int(Mode.STATIC))

    def prepare(self, lengths, splits):
        """The reference benchmark's STATIC_CPU entry (benchmarks/bench_decode.py:14-30): host
        LPT and upload for this call's lengths, the R1 plan on the device, the lists
        installed over it.  The engine must be built with force_mode R1."""
        self.plan_lists(lengths, splits)
        self.engine.prepare()
        self.apply()
