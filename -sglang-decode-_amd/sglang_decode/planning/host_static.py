"""Host-planned STATIC schedule: the "strong static" baseline of the reference's benchmark.

benchmarks/bench_decode.py:14-30 of the reference plans the STATIC lists on the host
(heap LPT over the records, planning/reference.py:57-67) on every call, builds the R1
plan on the device for the common records, then replaces only the dispatch metadata:
static_head / static_next uploaded, mode forced to STATIC.

Here the records and the LPT are built in C++ (``sgd_host_static_plan``) straight from
the lengths and split counts, into pinned host staging buffers uploaded with
asynchronous copies on the current stream; ``prepare`` is the reference's per-call
boundary (LPT + upload + R1 build + STATIC forced).
"""
import ctypes

import numpy as np
import torch

from .. import _lib
from ..config import Mode


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
    """Host LPT lists of one engine's plan, uploaded from pinned host staging.

    ``plan_lists`` runs split + heap LPT in C++ (``sgd_host_static_plan``) straight from
    the lengths and split counts and copies the lists asynchronously, on the current
    stream, into the plan's own static_head / static_next (an R1 plan build never writes
    them, so they survive ``prepare()``); ``apply`` then only forces STATIC, one device
    op a hipGraph can capture.  Two staging buffers alternate, so a call waits only for
    the upload two calls back -- long done -- never for the previous one, and the host
    keeps running ahead of the GPU."""

    def __init__(self, engine):
        self.engine = engine
        p = engine.plan
        pinned = p.device.type == "cuda"
        self._staging = [(torch.empty(p.static_head.shape, dtype=torch.int32, pin_memory=pinned),
                          torch.empty(p.static_next.shape, dtype=torch.int32, pin_memory=pinned)) for _ in range(2)]
        self._uploaded = [torch.cuda.Event() if pinned else None for _ in range(2)]
        self._pending = [False, False]
        self._turn = 0
        self._record_count = np.zeros(1, dtype=np.int32)

    def plan_lists(self, lengths, splits):
        """Host LPT for these lengths/splits (ValueError beyond the capacities), written to
        a pinned staging pair and copied into the plan's lists on the current stream."""
        c = self.engine.config
        lengths = np.ascontiguousarray(lengths, dtype=np.int32)
        splits = np.ascontiguousarray(splits, dtype=np.int32)
        if lengths.shape != splits.shape or lengths.ndim != 1 or len(lengths) > c.batch_capacity:
            raise ValueError(f"host static plan: lengths and splits must be two equal 1-D lists of at most "
                             f"{c.batch_capacity} requests")
        i = self._turn
        self._turn ^= 1
        if self._pending[i]:
            self._uploaded[i].synchronize()
        heads, nxt = self._staging[i]
        p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
        _lib.check(_lib.lib().sgd_host_static_plan(
            p(lengths), p(splits), len(lengths), c.max_splits, c.max_context, c.block_kv, c.kv_heads, c.workers,
            c.task_capacity, p(heads.numpy()), p(nxt.numpy()), p(self._record_count)), "host static plan")
        plan = self.engine.plan
        plan.static_head.copy_(heads, non_blocking=True)
        plan.static_next.copy_(nxt, non_blocking=True)
        if self._uploaded[i] is not None:
            self._uploaded[i].record()
            self._pending[i] = True

    def apply(self):
        """After an R1 ``prepare()``: run the uploaded lists (force STATIC; device op only)."""
        self.engine.plan.mode.fill_(int(Mode.STATIC))

    def prepare(self, lengths, splits):
        """The reference benchmark's STATIC_CPU entry (benchmarks/bench_decode.py:14-30): host
        LPT and upload for this call's lengths, the R1 plan on the device, STATIC forced over
        it.  The engine must be built with force_mode R1 and its own prepare() unpatched."""
        self.plan_lists(lengths, splits)
        self.engine.prepare()
        self.apply()
