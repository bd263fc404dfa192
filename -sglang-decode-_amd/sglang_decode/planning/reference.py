"""Host-side planning API (the CPU planning spec of src/sglang_decode/planning/reference.py:6-76).

The names, arguments and results are the reference's; the computation is this
module's own: each stage is one pass over numpy arrays of the batch, and the LPT
lists come from the native library's C++ heap planner.

* ``split_records(lengths, splits, config)`` -> (records, counts, offsets).  A request
  of L tokens asking for S splits is cut into chunks of c = ceil(ceil(L/S)/32)*32
  tokens, n = ceil(L/c) of them (0 when L is 0); record i of the request covers
  [i*c, min((i+1)*c, L)) and weighs ceil(tokens/block_kv).  Records are numbered
  request-major.  Shapes or values outside the configuration raise ValueError.
* ``bucket_order(records)`` -> record ids ordered by decreasing bucket, bucket(w) =
  bit length of w-1 (= ceil(log2 w)), ties kept in id order.
* ``make_packs(records, order, groups, workers, pack_limit=4)`` -> [(first task,
  tasks)]: per bucket of the order, its tasks (records x groups, consecutive) are cut
  into packs of width min(pack_limit, max(1, max_weight >> bucket)) except for the
  last `workers` tasks (rounded so that the packs are whole), which stay single.
* ``greedy_static(records, groups, workers)`` -> per-worker task lists: tasks by
  decreasing weight then id, each given to the worker with the least (load, id).
* ``lists_to_links`` / ``validate_plan``: the lists as static_head/static_next arrays,
  and the plan invariants (order a permutation, packs covering every task once, no two
  tasks on one (request, split, head) slot).
"""
from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class Record:
    request: int
    split: int
    begin: int
    end: int
    weight: int


def _ceil_div(a, b):
    return -(-a // b)


def _record_arrays(lengths, splits, config):
    """Columns (request, split, begin, end, weight) of the batch's records plus the
    per-request counts and offsets, as int64 numpy arrays."""
    length = np.asarray(lengths, dtype=np.int64).reshape(-1)
    want = np.asarray(splits, dtype=np.int64).reshape(-1)
    if length.shape != want.shape:
        raise ValueError(f"split_records: {length.size} lengths but {want.size} split counts")
    if length.size > config.batch_capacity:
        raise ValueError(f"split_records: batch {length.size} exceeds batch_capacity {config.batch_capacity}")
    bad = (length < 0) | (length > config.max_context) | (want < 1) | (want > config.max_splits)
    if bad.any():
        r = int(np.flatnonzero(bad)[0])
        raise ValueError(f"split_records: request {r} has length {int(length[r])} (allowed 0..{config.max_context}) "
                         f"and {int(want[r])} splits (allowed 1..{config.max_splits})")
    chunk = _ceil_div(_ceil_div(length, want), 32) * 32
    count = np.where(chunk > 0, _ceil_div(length, np.maximum(chunk, 1)), 0)
    offsets = np.concatenate(([0], np.cumsum(count)))
    request = np.repeat(np.arange(length.size), count)
    split = np.arange(int(offsets[-1])) - offsets[request]
    begin = split * chunk[request]
    end = np.minimum(begin + chunk[request], length[request])
    weight = _ceil_div(end - begin, config.block_kv)
    return (request, split, begin, end, weight), count, offsets


def split_records(lengths, requested_splits, config):
    cols, count, offsets = _record_arrays(lengths, requested_splits, config)
    records = [Record(*row) for row in zip(*(c.tolist() for c in cols))]
    return records, count.tolist(), offsets.tolist()


def _weights(records):
    return np.fromiter((r.weight for r in records), dtype=np.int64, count=len(records))


def _buckets(weight):
    """Bit length of w - 1 for every weight (0 for w <= 1)."""
    v = np.maximum(np.asarray(weight, dtype=np.int64) - 1, 0)
    bits = np.zeros_like(v)
    while v.any():
        bits += v > 0
        v >>= 1
    return bits


def bucket_order(records):
    return np.argsort(-_buckets(_weights(records)), kind="stable").tolist()


def make_packs(records, order, groups, workers, pack_limit=4):
    if not records:
        return []
    weight = _weights(records)
    bucket = _buckets(weight)[np.asarray(order, dtype=np.int64)]
    top = int(weight.max())
    # runs of equal bucket along the order: [start, stop) in records
    cuts = np.flatnonzero(np.diff(bucket)) + 1
    starts = np.concatenate(([0], cuts))
    stops = np.concatenate((cuts, [bucket.size]))
    firsts, widths = [], []
    for start, stop, b in zip(starts.tolist(), stops.tolist(), bucket[starts].tolist()):
        tasks = (stop - start) * groups
        width = min(pack_limit, max(1, top >> b))
        wide = max(0, tasks - workers) // width * width
        base = start * groups
        firsts.append(base + np.arange(0, wide, width))
        widths.append(np.full(wide // width, width))
        firsts.append(base + np.arange(wide, tasks))
        widths.append(np.ones(tasks - wide, dtype=np.int64))
    first, width = np.concatenate(firsts), np.concatenate(widths)
    return list(zip(first.tolist(), width.tolist()))


def greedy_static(records, groups, workers):
    from .host_static import host_static_lists
    tasks = len(records) * groups
    heads, nxt = host_static_lists(_weights(records), groups, workers, max(tasks, 1))
    lists = []
    for head in heads.tolist():
        chain, t = [], head
        while t >= 0:
            chain.append(t)
            t = int(nxt[t])
        lists.append(chain)
    return lists


def lists_to_links(lists, workers, task_capacity):
    """Per-worker lists -> (static_head[workers], static_next[task_capacity]), -1 terminated."""
    heads = np.full(workers, -1, dtype=np.int64)
    links = np.full(task_capacity, -1, dtype=np.int64)
    for worker, chain in enumerate(lists):
        if chain:
            heads[worker] = chain[0]
            links[np.asarray(chain[:-1], dtype=np.int64)] = chain[1:]
    return heads.tolist(), links.tolist()


def validate_plan(records, order, packs, groups):
    n = len(records)
    if sorted(order) != list(range(n)):
        raise AssertionError("validate_plan: the order must list every record exactly once")
    covered = np.zeros(n * groups, dtype=np.int64)
    for first, count in packs:
        covered[first:first + count] += 1
    if covered.size and (covered != 1).any():
        raise AssertionError(f"validate_plan: task {int(np.flatnonzero(covered != 1)[0])} is scheduled "
                             f"{int(covered[covered != 1][0])} times")
    if sum(count for _, count in packs) != n * groups:
        raise AssertionError("validate_plan: the packs schedule more tasks than exist")
    ordered = np.asarray(order, dtype=np.int64)
    key = {(records[ordered[t // groups]].request, records[ordered[t // groups]].split, t % groups)
           for t in range(n * groups)}
    if len(key) != n * groups:
        raise AssertionError("validate_plan: two tasks write one (request, split, head) slot")
