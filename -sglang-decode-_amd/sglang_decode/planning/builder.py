"""Device plan build: fixed launches, no allocation, no host readback.

``build_plan(plan, force_mode)`` has the contract of
src/sglang_decode/planning/builder.py:6-33: count/scan, records, mode/order/packs
and -- only when STATIC is forced or a policy rule can select it (decided at
capture time, never from a device scalar) -- the device LPT lists.  A forced R0
stops after the count/scan with mode 0 and no packs.

By default the whole sequence is ONE launch of the fused plan kernel; pass
``fused=False`` to issue the four stage launches of the reference instead (same
results; used by the parity tests of each stage).
"""
from ..kernels import plan as K


def build_plan(plan, force_mode=-1, *, fused=True, counters=None, csr_metadata=None):
    """``csr_metadata`` = (kv_indptr, num_kv_splits, batch): the fused
    build reads the step's lengths, split counts and batch from them (no copies into the
    plan beforehand); the staged path makes those copies itself."""
    force_mode = int(force_mode)
    run_greedy = force_mode == 2 or any_static_rule(plan)
    if fused:
        K.fused_build(plan, force_mode, run_greedy, counters, csr_metadata)
        plan.dispatch_valid = True
        return
    plan.dispatch_valid = False  # the stage launches do not write the dispatch table
    if counters is not None:
        counters.zero_()
    if csr_metadata is not None:
        indptr, splits, batch = csr_metadata
        plan.lengths[:batch].copy_(indptr[1:batch + 1] - indptr[:batch])
        plan.splits[:batch].copy_(splits[:batch])
        plan.active.fill_(batch)
    K.count_scan(plan)
    if force_mode == 0:
        plan.mode.fill_(0)
        plan.num_packs.zero_()
        return
    K.emit_records(plan)
    K.order_and_packs(plan, force_mode)
    if run_greedy:
        K.greedy_lists(plan)


def any_static_rule(plan):
    # Capture-time metadata set by the runtime; never inspect a device scalar here.
    return getattr(plan, "has_static_rule", False)
