"""Host-side planning: the CPU planning API and the strong host static baseline.

Same functions and results as src/sglang_decode/planning/reference.py:6-76:

* ``split_records`` -- chunk = ceil(ceil(L/S)/32)*32, count = ceil(L/chunk), one
  record (request, split, begin, end, weight=ceil((end-begin)/block_kv)) per split,
  raising ValueError on capacity violations (reference.py:15-30);
* ``bucket_order`` -- records stably ordered heaviest ceil-log2 bucket first
  (reference.py:33-34);
* ``make_packs`` -- per bucket, reserve one worker wave of singleton tasks and
  pack the rest ``width = min(limit, max(1, max_w >> bucket))`` wide
  (reference.py:37-54);
* ``greedy_static`` -- longest-processing-time lists with (load, worker) tie
  breaks (reference.py:57-67).  ``host_static_lists`` returns the same lists as
  the device's ``static_head``/``static_next`` arrays, computed by the native
  library's C++ heap planner (used for the host-static variant that uploads its
  lists, benchmarks/bench_decode.py:14-30);
* ``validate_plan`` -- coverage and slot uniqueness (reference.py:70-76).
"""
from dataclasses import dataclass
import heapq


@dataclass(frozen=True)
class Record:
    request: int
    split: int
    begin: int
    end: int
    weight: int


def split_records(lengths, requested_splits, config):
    if len(lengths) != len(requested_splits) or len(lengths) > config.batch_capacity:
        raise ValueError("batch/split shape exceeds the capture contract")
    records, offsets, counts = [], [0], []
    for request, (length, splits) in enumerate(zip(lengths, requested_splits)):
        if not 0 <= length <= config.max_context or not 1 <= splits <= config.max_splits:
            raise ValueError("invalid length or split count")
        chunk = -(-(-(-length // splits)) // 32) * 32
        count = -(-length // chunk) if chunk else 0
        counts.append(count)
        for split in range(count):
            begin = split * chunk
            end = min(begin + chunk, length)
            records.append(Record(request, split, begin, end,
                                  -(-(end - begin) // config.block_kv)))
        offsets.append(len(records))
    return records, counts, offsets


def _bucket(weight):
    return (weight - 1).bit_length()


def bucket_order(records):
    return sorted(range(len(records)), key=lambda i: -_bucket(records[i].weight))


def make_packs(records, order, groups, workers, pack_limit=4):
    """Pack within one bucket; reserve a full worker wave of singleton tasks."""
    packs = []
    max_weight = max((r.weight for r in records), default=1)
    first = 0
    while first < len(order):
        bucket = _bucket(records[order[first]].weight)
        last = first
        while last < len(order) and _bucket(records[order[last]].weight) == bucket:
            last += 1
        tasks = (last - first) * groups
        width = min(pack_limit, max(1, max_weight >> bucket))
        packed = max(0, tasks - workers) // width * width
        base = first * groups
        packs.extend((base + i, width) for i in range(0, packed, width))
        packs.extend((base + i, 1) for i in range(packed, tasks))
        first = last
    return packs


def greedy_static(records, groups, workers):
    """LPT lists: tasks by (-weight, task id), each to the least (load, worker)."""
    tasks = sorted(range(len(records) * groups), key=lambda t: (-records[t // groups].weight, t))
    heap = [(0, w) for w in range(workers)]
    lists = [[] for _ in range(workers)]
    for task in tasks:
        load, worker = heapq.heappop(heap)
        lists[worker].append(task)
        heapq.heappush(heap, (load + records[task // groups].weight, worker))
    return lists


def lists_to_links(lists, workers, task_capacity):
    """Per-worker lists -> (static_head[workers], static_next[task_capacity]), -1 terminated."""
    heads = [-1] * workers
    links = [-1] * task_capacity
    for worker, tasks in enumerate(lists):
        if tasks:
            heads[worker] = tasks[0]
        for left, right in zip(tasks, tasks[1:]):
            links[left] = right
    return heads, links


def validate_plan(records, order, packs, groups):
    if sorted(order) != list(range(len(records))):
        raise AssertionError("order is not a permutation of the records")
    tasks = [task for first, count in packs for task in range(first, first + count)]
    if sorted(tasks) != list(range(len(records) * groups)):
        raise AssertionError("packs do not cover every task exactly once")
    slots = {(records[order[t // groups]].request, records[order[t // groups]].split,
              t % groups) for t in tasks}
    if len(slots) != len(tasks):
        raise AssertionError("two tasks write the same (request, split, head) slot")
