"""Device plan stages (thin wrappers over the C ABI; the kernels live in csrc/plan.hip).

One function per reference stage (src/sglang_decode/kernels/plan.py) plus the
fused single-launch build used by ``planning.builder.build_plan``.
"""
import ctypes

import torch

from .. import _lib
from .._lib import check, ptr


def _s(plan):
    return _lib.stream_handle(plan.device)


def count_scan(plan):
    """kernels/plan.py:7-27."""
    c = plan.config
    check(_lib.lib().sgd_count_scan(
        ptr(plan.lengths), ptr(plan.splits), ptr(plan.active), ptr(plan.counts), ptr(plan.offsets),
        ptr(plan.chunk), ptr(plan.record_count), ptr(plan.error), c.batch_capacity, c.max_splits,
        c.max_context, _s(plan)), "count_scan")


def emit_records(plan):
    """kernels/plan.py:30-45."""
    c = plan.config
    check(_lib.lib().sgd_emit_records(
        ptr(plan.lengths), ptr(plan.counts), ptr(plan.offsets), ptr(plan.chunk), ptr(plan.request),
        ptr(plan.split), ptr(plan.begin), ptr(plan.end), ptr(plan.weight), c.batch_capacity,
        c.max_splits, c.block_kv, _s(plan)), "emit_records")


def order_and_packs(plan, force_mode=-1):
    """kernels/plan.py:48-100."""
    c = plan.config
    check(_lib.lib().sgd_order_and_packs(
        ptr(plan.weight), ptr(plan.record_count), ptr(plan.order), ptr(plan.pack_first),
        ptr(plan.pack_count), ptr(plan.num_packs), ptr(plan.mode), ptr(plan.rules),
        plan.rule_count, int(force_mode), c.kv_heads, c.workers, c.buckets, c.record_capacity,
        _s(plan)), "order_and_packs")


def greedy_lists(plan):
    """kernels/plan.py:103-135 (runs only when plan.mode == 2)."""
    c = plan.config
    check(_lib.lib().sgd_greedy_lists(
        ptr(plan.weight), ptr(plan.record_count), ptr(plan.mode), ptr(plan.static_head),
        ptr(plan.static_next), c.kv_heads, c.workers, c.record_capacity, _s(plan)),
        "greedy_lists")


def fused_build(plan, force_mode=-1, run_greedy=False, counters=None, csr_metadata=None):
    """All stages in one launch; optionally clears ``counters`` (int32) in the same launch.
    ``csr_metadata`` = (kv_indptr,
    num_kv_splits, batch): the lengths, split counts and active count come from the step's
    CSR metadata inside the launch (and are stored to the plan), instead of from copies
    made into the plan beforehand (integrations/sglang_backend.py:98-99)."""
    n = 0 if counters is None else counters.numel()
    if csr_metadata is None:
        check(_lib.lib().sgd_build_plan(ctypes.byref(plan.c_struct()), int(force_mode),
                                        int(bool(run_greedy)), ptr(counters), n, _s(plan)), "build_plan")
        return
    indptr, splits, batch = csr_metadata
    batch = int(batch)
    for name, t, need in (("kv_indptr", indptr, batch + 1), ("num_kv_splits", splits, batch)):
        if t.dtype != torch.int32 or t.device != plan.device or t.dim() != 1 or t.shape[0] < need:
            raise ValueError(f"build_plan_csr: {name} must be int32 [>= {need}] on the plan's device")
    if not 0 <= batch <= plan.config.batch_capacity:
        raise ValueError(f"build_plan_csr: batch {batch} outside [0, {plan.config.batch_capacity}]")
    indptr, splits = indptr.contiguous(), splits.contiguous()
    check(_lib.lib().sgd_build_plan_csr(ctypes.byref(plan.c_struct()), ptr(indptr), ptr(splits), batch,
                                        int(force_mode), int(bool(run_greedy)), ptr(counters), n, _s(plan)),
          "build_plan_csr")
