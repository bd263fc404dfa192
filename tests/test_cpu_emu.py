"""The library's kernels executed on the CPU (tests/cpu_emu) under AddressSanitizer.

Each thread of a workgroup runs as a fiber.  Cross-lane operations are evaluated over the
lanes that reach them, and reading a lane that is switched off is an error.  Every
buffer is an exact-size host allocation, so an access outside a buffer, the dynamic LDS
block or a static LDS array aborts the run with the kernel, workgroup and thread named.

What this pins:
* The GPU memory fault of the sweep's seed 15 (max_splits 1, lengths [10, 15490], D4,
  256 workers; 4 tasks, the heavy record in weight bucket 7).  The fused plan build's
  pack-table and dispatch-table loops run one task per lane, so lanes past the last task
  are switched off.  bucket_at() read the bucket tables with v_readlane from per-lane
  registers, and the compiler loads those registers inside the loop, so bucket 7's entry
  was read from lane 7's stale registers.  The garbage pack index was then stored
  through (pack_first/pack_count/dispatch).  The executor rejects exactly that
  inactive-lane read, so these cases fail if the pattern comes back.
* The held sweep draws and the long-task draws run in bounds on every kernel that takes
  their shape, match the FP32 oracle (2e-2 abs / 1e-2 rel), build the oracle's plan
  bit-exactly and leave the claim counters at zero.
* The entry points outside the engine's path -- the upstream comparator and the
  no-allocation entry with its static device array -- run in bounds as well.
"""
import json
import os
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
EMU = os.path.join(HERE, "cpu_emu")
if EMU not in sys.path:
    sys.path.insert(0, EMU)


@pytest.fixture(scope="module")
def asan_build():
    import build as B
    return B.build(asan=True)


EMU_JOBS = max(1, min(6, (os.cpu_count() or 2) - 2))  # executor processes at once


def _run(cases, **kw):
    """Each case in an executor process of its own, up to EMU_JOBS at a time (the cases are
    independent); the rows come back in case order."""
    import concurrent.futures
    import run_cases as R
    with concurrent.futures.ThreadPoolExecutor(min(EMU_JOBS, len(cases))) as pool:
        results = list(pool.map(lambda case: R.spawn([case], **kw), cases))
    rc = next((r for r, _, _ in results if r != 0), 0)
    err = "".join(e for _, _, e in results)
    rows = [json.loads(line) for _, out, _ in results for line in out.splitlines() if line.startswith("{")]
    return rc, rows, err



def _assert_clean(rc, rows, err, expected_rows):
    assert rc == 0, f"executor run failed (rc {rc}):\n{err[-4000:]}"
    assert "ERROR: AddressSanitizer" not in err, err[-4000:]
    assert len(rows) == expected_rows, (len(rows), err[-2000:])
    for r in rows:
        assert r["violations"] == 0 and r["nans"] == 0, r
        assert r["tail"] == 0.0, r        # rows past the batch are exact zeros
        assert r["plan_ok"], r            # plan bit-exact against the oracle
        assert r["counters"] == [0, 0], r  # claim / finished counters back at zero


# (seed, kernels): the held max_splits-1 draws, then draws with the longest tasks.
SWEEP = [(15, ["generic", "mfma", "valu"]), (16, ["generic"]), (17, ["generic", "mfma"]),
         (21, ["generic", "mfma", "valu"]), (31, ["generic"]), (8, ["valu"]), (2, ["mfma"])]


# sweep draws at head_dim 64 and 256 with groups <= 4: the VALU kernel's other tile
# geometries (32- and 8-token tiles), CSR and paged, one worker and many
SWEEP_HEAD_DIMS = [0, 11, 28, 29, 36, 37]


# sweep draws at head_dim 64 and 256 on the MFMA kernel: group 8 CSR (D 64 and 256), group 8
# paged with one request, groups 4 and 2 paged at D 256 (the 16-token tiles)
SWEEP_MFMA_HEAD_DIMS = [4, 16, 27, 28, 37]


def test_mfma_head_dims_in_bounds(asan_build):
    cases = [{"sweep": s, "kernels": ["mfma"]} for s in SWEEP_MFMA_HEAD_DIMS]
    rc, rows, err = _run(cases)
    _assert_clean(rc, rows, err, len(SWEEP_MFMA_HEAD_DIMS))


# sweep draws with pages of 12 tokens (mapped by division): group 2 (D 128) and group 4
# (D 256, 4096-token rows) on both tuned kernels, group 16 (D 128) on the MFMA one
SWEEP_PAGES_NOT_POW2 = [(23, ["mfma", "valu"]), (73, ["mfma", "valu"]), (22, ["mfma"])]


def test_pages_not_a_power_of_two_in_bounds(asan_build):
    cases = [{"sweep": s, "kernels": k} for s, k in SWEEP_PAGES_NOT_POW2]
    rc, rows, err = _run(cases)
    _assert_clean(rc, rows, err, sum(len(k) for _, k in SWEEP_PAGES_NOT_POW2))


def test_valu_head_dims_in_bounds(asan_build):
    cases = [{"sweep": s, "kernels": ["valu"]} for s in SWEEP_HEAD_DIMS]
    rc, rows, err = _run(cases)
    _assert_clean(rc, rows, err, len(SWEEP_HEAD_DIMS))


def test_selective_merge_strides_in_bounds(asan_build):
    """sgd_merge_splits_min with more rows than resident workgroups (the executor reports
    one per CU, 256 here; 512 rows) at every head dim: merged rows bitwise equal to
    sgd_merge_splits, skipped rows untouched, NaN on a plan error, all in bounds."""
    cases = [{"merge_min": [64, 8, 64, d, 2]} for d in (64, 128, 256)] + [{"merge_min": [64, 8, 16, 128, 17]}]
    rc, rows, err = _run(cases)
    assert rc == 0 and "ERROR: AddressSanitizer" not in err, err[-4000:]
    assert len(rows) == len(cases), err[-2000:]
    for r in rows:
        assert r["merged_equal"] and r["skipped_untouched"] and r["error_nan"], r


def test_sweep_draws_in_bounds(asan_build):
    cases = [{"sweep": s, "kernels": k} for s, k in SWEEP]
    rc, rows, err = _run(cases)
    _assert_clean(rc, rows, err, sum(len(k) for _, k in SWEEP))


def test_small_batch_every_mode_and_kernel(asan_build):
    """Batch 4 at 8/2 heads: every schedule on every kernel, and the reversed workgroup
    order (the dynamic schedules then hand the claims to other workers)."""
    kernels, modes = ["generic", "mfma", "valu"], [0, 1, 2, 3, 4]
    case = [{"workload": "c1", "kernels": kernels, "modes": modes}]
    for env in (None, {"EMU_ORDER": "reverse"}):
        rc, rows, err = _run(case, env_extra=env)
        _assert_clean(rc, rows, err, len(kernels) * len(modes))


def test_few_workers_walk_long_task_chains(asan_build):
    """3 to 5 workers, so every worker runs many tasks in a row: the next-task search that
    the last wave of the valu and mfma kernels makes while the other waves finish (the
    claim, the entry or record, the first tiles' page/slot indices, left in LDS by task
    parity) is taken on every task boundary -- new units and packs of several tasks,
    CSR and paged, every schedule -- in bounds and against the oracle."""
    cases = [{"workload": "c1", "workers": 3, "kernels": ["valu", "mfma"], "modes": [0, 1, 2, 3, 4]},
             {"workload": "c4", "workers": 5, "requests": 1, "kernels": ["mfma"], "modes": [4]},
             {"workload": "c2", "workers": 5, "requests": 2, "kernels": ["valu"], "modes": [3]}]
    rc, rows, err = _run(cases)
    _assert_clean(rc, rows, err, 10 + 1 + 1)


def test_upstream_comparator_and_no_alloc_entry_in_bounds(asan_build):
    """The two entry points outside the engine's path.  sgd_upstream_decode (the upstream
    two-stage split-KV comparator): empty, 1-token and 700-token rows over 16 splits, a
    3000-token row over 4 (fp16), equal rows with one split -- output and every non-empty
    split slot against the oracle.  sgd_decode_noalloc (plan tables, counters and split
    slots in the library's static array): two calls in a row, the second smaller, CSR (D1)
    and paged group 8 (D4), each bitwise equal to the allocating entry points."""
    cases = [{"upstream": [[0, 1, 17, 33, 257, 513, 700], 16]},
             {"upstream": [[3000, 5, 129], 4], "dtype": "float16"},
             {"upstream": [[64] * 5, 1]},
             {"noalloc": "c1", "batches": [[4, 1], [2, 3]], "mode": 3},
             {"noalloc": "c4", "batches": [[2, 16], [1, 32]], "mode": 4}]
    rc, rows, err = _run(cases)
    assert rc == 0, f"executor run failed (rc {rc}):\n{err[-4000:]}"
    assert "ERROR: AddressSanitizer" not in err, err[-4000:]
    assert len(rows) == len(cases), (len(rows), err[-2000:])
    for r in rows:
        if r["case"] == "upstream":
            assert r["violations"] == 0 and r["slot_violations"] == 0 and r["nans"] == 0, r
            assert r["slots"] > 0, r
        else:
            assert len(r["calls"]) == 2, r
            for call in r["calls"]:
                assert call["bitwise"] and call["violations"] == 0 and call["tail"] == 0.0, r


def test_executor_reports_out_of_bounds(asan_build):
    """The harness itself: an output buffer one row short makes the merge store past it,
    and the run aborts with AddressSanitizer's report naming the kernel."""
    import build as B
    env = dict(os.environ, LD_PRELOAD=B.asan_runtime(), ASAN_OPTIONS="detect_leaks=0:abort_on_error=1")
    code = r"""
import ctypes, sys
sys.path.insert(0, %r)
import numpy as np
import driver as D
emu = D.Emu(asan=True)
bcap, hq, d, smax = 2, 1, 64, 1
partial = emu.array((bcap, hq, smax, d), np.float32, 0.5)
lse = emu.array((bcap, hq, smax), np.float32, 0.0)
counts = emu.array((bcap,), np.int32, 1)
active = emu.array((1,), np.int32, bcap)
error = emu.array((1,), np.int32, 0)
out = emu.array((bcap * hq * d - 1,), np.uint16)   # one element short
emu.lib.sgd_merge_splits(D.ptr(partial), D.ptr(lse), D.ptr(counts), D.ptr(active), D.ptr(error), D.ptr(out),
                         bcap, hq, d, smax, 0, None)
print("no report")
""" % EMU
    import subprocess
    p = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=300)
    assert p.returncode != 0, p.stdout
    assert "heap-buffer-overflow" in p.stderr, p.stderr[-3000:]
    assert "k_merge" in p.stderr, p.stderr[-3000:]


def test_static_lists_rounds_match_sequential_lpt(asan_build):
    """The device STATIC lists are assigned in rounds of equal-weight tasks (csrc/plan.hip
    stage_greedy_lists); on 80 random plans -- uniform, spread and mostly-light weights
    with a few heavy records (loads far apart: rounds of a few tasks), 1 to 512 workers --
    the walked lists equal the oracle's one-task-at-a-time (load, worker) argmin LPT
    (kernels/plan.py:103-135), in bounds under AddressSanitizer."""
    rc, rows, err = _run([{"lpt": 80, "seed": 3}])
    assert rc == 0, err[-4000:]
    assert "ERROR: AddressSanitizer" not in err, err[-4000:]
    assert rows and rows[0]["mismatches"] == 0, rows
