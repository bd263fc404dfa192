"""ORACLE (test infrastructure only): ctypes front end for oracle/plan_spec.c.

Each function returns plain Python lists so tests can compare them directly with
device buffers.  Builds liboracle_plan.so with the committed Makefile on first
use when it is missing (gcc only; no GPU).
"""
import ctypes
import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_plan.so")
_lib = None


def build():
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle_plan.so"], check=True)


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
    return _lib


def _arr(values, n=None):
    n = len(values) if n is None else n
    buf = (ctypes.c_int32 * max(n, 1))()
    for i, v in enumerate(values[:n]):
        buf[i] = int(v)
    return buf


def count_scan(lengths, splits, active, bcap, smax, max_context):
    """kernels/plan.py:7-27.  Returns dict(counts, offsets, chunk, record_count, error)."""
    lib = _load()
    counts, offsets, chunk = _arr([], bcap), _arr([], bcap + 1), _arr([], bcap)
    rc, err = ctypes.c_int32(), ctypes.c_int32()
    lib.orc_count_scan(_arr(lengths, bcap), _arr(splits, bcap), ctypes.c_int32(active),
                       ctypes.c_int32(bcap), ctypes.c_int32(smax), ctypes.c_int32(max_context),
                       counts, offsets, chunk, ctypes.byref(rc), ctypes.byref(err))
    return dict(counts=list(counts)[:bcap], offsets=list(offsets)[:bcap + 1],
                chunk=list(chunk)[:bcap], record_count=rc.value, error=err.value)


def emit_records(lengths, counts, offsets, chunk, bcap, smax, tile, record_capacity):
    """kernels/plan.py:30-45.  Returns the five SoA arrays (length record_capacity, 0-filled)."""
    lib = _load()
    out = [_arr([], record_capacity) for _ in range(5)]
    lib.orc_emit_records(_arr(lengths, bcap), _arr(counts, bcap), _arr(offsets, bcap + 1),
                         _arr(chunk, bcap), ctypes.c_int32(bcap), ctypes.c_int32(smax),
                         ctypes.c_int32(tile), *out)
    names = ("request", "split", "begin", "end", "weight")
    return {k: list(v)[:record_capacity] for k, v in zip(names, out)}


def order_and_packs(weight, total, rules, force, hkv, workers, buckets, record_capacity):
    """kernels/plan.py:48-100.  rules: iterable of 5-int rows."""
    lib = _load()
    task_capacity = record_capacity * hkv
    flat = [int(x) for row in rules for x in row]
    order, first, count = _arr([], record_capacity), _arr([], task_capacity), _arr([], task_capacity)
    num_packs, mode = ctypes.c_int32(), ctypes.c_int32()
    lib.orc_order_and_packs(_arr(weight, max(total, 1)), ctypes.c_int32(total), _arr(flat),
                            ctypes.c_int32(len(flat) // 5), ctypes.c_int32(force),
                            ctypes.c_int32(hkv), ctypes.c_int32(workers), ctypes.c_int32(buckets),
                            order, first, count, ctypes.byref(num_packs), ctypes.byref(mode))
    n = num_packs.value
    return dict(order=list(order)[:total], pack_first=list(first)[:n],
                pack_count=list(count)[:n], num_packs=n, mode=mode.value)


def greedy_lists(weight, total, mode, hkv, workers, task_capacity):
    """kernels/plan.py:103-135 (device LPT).  Returns (heads, next) with untouched next = -2."""
    lib = _load()
    heads = _arr([-2] * workers)
    nxt = _arr([-2] * task_capacity)
    lib.orc_greedy_lists(_arr(weight, max(total, 1)), ctypes.c_int32(total), ctypes.c_int32(mode),
                         ctypes.c_int32(hkv), ctypes.c_int32(workers), heads, nxt)
    return list(heads)[:workers], list(nxt)[:task_capacity]


def greedy_static(weight, total, hkv, workers, task_capacity):
    """planning/reference.py:57-67 as linked lists (bench_decode.py:16-30 conversion)."""
    lib = _load()
    heads, nxt = _arr([], workers), _arr([], task_capacity)
    lib.orc_greedy_static(_arr(weight, max(total, 1)), ctypes.c_int32(total), ctypes.c_int32(hkv),
                          ctypes.c_int32(workers), ctypes.c_int32(task_capacity), heads, nxt)
    return list(heads)[:workers], list(nxt)[:task_capacity]


def walk_lists(heads, nxt):
    """Expand (head, next) linked lists into per-worker task lists."""
    lists = []
    limit = len(nxt)
    for h in heads:
        items, t = [], h
        while 0 <= t < limit:
            items.append(t)
            t = nxt[t]
            if len(items) > limit:
                raise AssertionError("cycle in static lists")
        lists.append(items)
    return lists


def merge_splits(partial, lse, counts, error, bcap, hq, d, smax):
    """kernels/merge.py:7-30 in float32.  partial/lse: numpy float32 arrays."""
    import numpy as np
    lib = _load()
    partial = np.ascontiguousarray(partial, dtype=np.float32)
    lse = np.ascontiguousarray(lse, dtype=np.float32)
    out = np.zeros((bcap, hq, d), dtype=np.float32)
    fp = ctypes.POINTER(ctypes.c_float)
    lib.orc_merge_splits(partial.ctypes.data_as(fp), lse.ctypes.data_as(fp), _arr(counts, bcap),
                         ctypes.c_int32(error), ctypes.c_int32(bcap), ctypes.c_int32(hq),
                         ctypes.c_int32(d), ctypes.c_int32(smax), out.ctypes.data_as(fp))
    return out


def full_plan(lengths, splits, active, cfg, rules=(), force=-1):
    """count_scan -> emit_records -> order_and_packs (-> greedy_lists when mode == 2),
    in the launch order of planning/builder.py:6-28.  cfg: object with the DecodeConfig fields."""
    bcap, smax = cfg.batch_capacity, cfg.max_splits
    e = bcap * smax
    cs = count_scan(lengths, splits, active, bcap, smax, cfg.max_context)
    plan = dict(cs)
    if int(force) == 0:
        plan.update(mode=0, num_packs=0)
        return plan
    rec = emit_records(lengths, cs["counts"], cs["offsets"], cs["chunk"], bcap, smax,
                       cfg.block_kv, e)
    plan.update(rec)
    total = cs["record_count"]
    buckets = ((cfg.max_context + cfg.block_kv - 1) // cfg.block_kv - 1).bit_length() + 1
    op = order_and_packs(rec["weight"][:total], total, rules, force, cfg.kv_heads,
                         cfg.workers, buckets, e)
    plan.update(op)
    if op["mode"] == 2:
        heads, nxt = greedy_lists(rec["weight"][:total], total, 2, cfg.kv_heads, cfg.workers,
                                  e * cfg.kv_heads)
        plan.update(static_head=heads, static_next=nxt)
    return plan
