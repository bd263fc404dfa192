"""Host-planned STATIC schedule: the "strong static" baseline of the reference's benchmark.

benchmarks/bench_decode.py:14-30 of the reference plans the STATIC lists on the host
(heap LPT over the records, planning/reference.py:57-67), builds the R1 plan on the
device for the common records, then replaces only the dispatch metadata: static_head /
static_next uploaded, mode forced to STATIC.  ``host_static_lists`` runs that LPT in
C++ (``sgd_host_static_lists``); ``HostStatic`` keeps the uploaded lists in fixed device
buffers so the replacement is three device operations that a hipGraph can capture
(two device-to-device copies and a fill kernel), with the host planning done when the
lengths change.
"""
import ctypes

import numpy as np
import torch

from .. import _lib
from ..config import Mode
from .reference import split_records


def host_static_lists(weights, kv_heads, workers, task_capacity):
    """(static_head [workers], static_next [task_capacity]) int32 host arrays, -1 terminated."""
    w = np.ascontiguousarray(np.asarray(weights, dtype=np.int32))
    heads = np.empty(workers, dtype=np.int32)
    nxt = np.empty(task_capacity, dtype=np.int32)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    _lib.check(_lib.lib().sgd_host_static_lists(p(w), len(w), kv_heads, workers, task_capacity,
                                                p(heads), p(nxt)), "host_static_lists")
    return heads, nxt


class HostStatic:
    """Fixed device copies of host LPT lists for one engine's plan."""

    def __init__(self, engine):
        self.engine = engine
        p = engine.plan
        self.heads = torch.full_like(p.static_head, -1)
        self.next = torch.full_like(p.static_next, -1)

    def plan_lists(self, lengths, splits):
        """Host LPT for these lengths/splits (raises ValueError beyond the capacities),
        uploaded to the fixed buffers on the current stream."""
        c = self.engine.config
        records, _, _ = split_records(lengths, splits, c)
        heads, nxt = host_static_lists([r.weight for r in records], c.kv_heads, c.workers,
                                       c.task_capacity)
        self.heads.copy_(torch.from_numpy(heads))
        self.next.copy_(torch.from_numpy(nxt))

    def apply(self):
        """After an R1 ``prepare()``: install the lists and force STATIC (device ops only)."""
        p = self.engine.plan
        p.static_head.copy_(self.heads)
        p.static_next.copy_(self.next)
        p.mode.fill_(int(Mode.STATIC))
