"""``benchmarks.workloads`` names (reference: benchmarks/workloads.py:5-50) over the
package's harness: the A/B/B64/uniform/holdout length sets, the split rule, the paged input
fixture and the plan-input upload.  Input bytes come from the package's seeded generators,
not the reference's device RNG, so they are equal in distribution, not in value."""
from sglang_decode import workloads as _w

WORKLOADS = {
    "A": [512] * 24 + [8192] * 8,
    "B": [256] * 24 + [1536] * 4 + [16384] * 4,
    "B64": ([256] * 24 + [1536] * 4 + [16384] * 4) * 2,
    "uniform": [1024] * 32,
    "holdout": [33, 255, 513, 1025, 3073, 8191, 16383],
}

split_hints = _w.split_hints


def make_inputs(config, lengths, seed=17, device="cuda", dtype=None):
    """(q [Bcap, Hq, D], k/v [pages, page, Hkv, D], page table [Bcap, max_pages], -1 padded)."""
    return _w.make_inputs(config, lengths, seed=seed, device=device, dtype=dtype)


def update_plan(engine, lengths):
    """Lengths, the harness's split counts and the active count into the engine's plan."""
    _w.update_plan(engine, lengths, split_hints(lengths, engine.config.max_splits))
