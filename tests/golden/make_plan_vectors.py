"""Write tests/golden/plan_vectors.json from the reference's own CPU planning spec.

Runs ONLY in the build container, where the reference checkout exists at
/root/reference.  It loads src/sglang_decode/planning/reference.py by file path
(the module imports nothing but dataclasses and heapq) and records, for each
seeded workload, the full sequences its functions return:

* split_records   -> records (request, split, begin, end, weight), counts, offsets
* bucket_order    -> order
* make_packs      -> packs for pack_limit 1 (D1) and 4 (D4)
* greedy_static   -> per-worker task lists

The reference's own tests pin these only by their lengths
(tests/unit/test_planning.py:9-48); these vectors pin the full sequences.  The
JSON holds inputs and outputs only.

Usage: python tests/golden/make_plan_vectors.py
"""
import importlib.util
import json
import os
import sys
import types

REF = "/root/reference/src/sglang_decode/planning/reference.py"
HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "-sglang-decode-_amd"))

from sglang_decode import workloads as W  # noqa: E402


def load_reference():
    spec = importlib.util.spec_from_file_location("_reference_planning_spec", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def cfg(bcap, smax, max_context, workers, hkv=8, block_kv=128):
    return types.SimpleNamespace(batch_capacity=bcap, max_splits=smax, max_context=max_context,
                                 workers=workers, kv_heads=hkv, block_kv=block_kv)


def case(ref, name, lengths, splits, c):
    records, counts, offsets = ref.split_records(lengths, splits, c)
    order = ref.bucket_order(records)
    packs1 = ref.make_packs(records, order, c.kv_heads, c.workers, pack_limit=1)
    packs4 = ref.make_packs(records, order, c.kv_heads, c.workers, pack_limit=4)
    lists = ref.greedy_static(records, c.kv_heads, c.workers)
    return dict(
        name=name, lengths=lengths, splits=splits,
        config=dict(batch_capacity=c.batch_capacity, max_splits=c.max_splits,
                    max_context=c.max_context, workers=c.workers, kv_heads=c.kv_heads,
                    block_kv=c.block_kv),
        records=[[r.request, r.split, r.begin, r.end, r.weight] for r in records],
        counts=counts, offsets=offsets, order=order,
        packs_d1=[list(p) for p in packs1], packs_d4=[list(p) for p in packs4],
        static_lists=lists)


def main():
    ref = load_reference()
    out = []
    # The reference's documented workloads (benchmarks/workloads.py:5-11) at its default
    # geometry (config.py:14-25: Bcap 64, Smax 16, max_context 32768, Hkv 8, 108 workers).
    documented = {
        "A": [512] * 24 + [8192] * 8,
        "B": [256] * 24 + [1536] * 4 + [16384] * 4,
        "B64": ([256] * 24 + [1536] * 4 + [16384] * 4) * 2,
        "holdout": [33, 255, 513, 1025, 3073, 8191, 16383],
        "edge": [0, 1, 17, 33, 257, 513],
    }
    for name, lengths in documented.items():
        for workers in (108, 256):
            c = cfg(64, 16, 32768, workers)
            out.append(case(ref, f"{name}/w{workers}", lengths, W.split_hints(lengths, 16), c))
    # Seeded benchmark configurations.
    for name in ("c1", "c2", "c3", "c4", "c5"):
        dc = W.config_for(name, workers=256)
        lengths = W.lengths_for(name)
        c = cfg(dc.batch_capacity, dc.max_splits, dc.max_context, dc.workers, dc.kv_heads)
        out.append(case(ref, f"{name}/w256", lengths, W.splits_for(name, lengths, dc), c))
    # C5's shrinking batches (first B rows survive, contexts +1 per step).
    base = W.c5_lengths()
    for step, batch in enumerate(W.C5_BATCHES):
        lengths = [x + step for x in base[:batch]]
        c = cfg(64, 16, 32768, 256)
        out.append(case(ref, f"c5_step{step}/w256", lengths, W.split_hints(lengths, 16), c))
    path = os.path.join(HERE, "plan_vectors.json")
    with open(path, "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print(f"wrote {len(out)} cases to {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
