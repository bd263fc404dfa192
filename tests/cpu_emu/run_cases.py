"""Runs decode cases on the CPU executor and checks them against the oracle (test
infrastructure).  Meant to run in its own process with the ASan build; ``spawn()``
starts it with clang's ASan runtime preloaded.

A case is a JSON object: {"lpt": trials} (random STATIC-list plans against the oracle's
sequential LPT, one JSON line with the mismatch count), {"sweep": seed} (the GPU sweep's draw of that seed, every
kernel that takes its shape), or {"workload": "c1".."c5", "modes": [...], "kernels":
[...], "requests": n} (a named configuration, optionally its first n requests).  One
JSON line per (case, kernel, mode) goes to stdout: violations of the 2e-2 abs / 1e-2 rel
tolerance, NaNs, nonzero rows past the batch, the plan compared bit-exactly with the
oracle, and the claim counters left at zero.

Two more case kinds drive the entry points outside the engine's path:
{"upstream": [lengths, max_splits], "dtype": ...} runs the upstream two-stage comparator
(sgd_upstream_decode) and checks its output and every non-empty split slot against the
oracle; {"noalloc": workload, "batches": [[n, shrink], ...], "mode": m} runs
sgd_decode_noalloc on consecutive calls (the first n requests, contexts divided by
shrink) and compares each bitwise with the allocating entry points on the same inputs.
"""
import json
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
TESTS = os.path.dirname(HERE)
ROOT = os.path.dirname(TESTS)


def spawn(cases, asan=True, timeout=900, env_extra=None):
    """Run ``cases`` in a child process; returns (returncode, stdout, stderr)."""
    import build as B
    env = dict(os.environ)
    if asan:
        env["LD_PRELOAD"] = B.asan_runtime()
        env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1:halt_on_error=1:allocator_may_return_null=1"
        env["ASAN_SYMBOLIZER_PATH"] = "/opt/rocm/llvm/bin/llvm-symbolizer"
    env.update(env_extra or {})
    cmd = [sys.executable, os.path.join(HERE, "run_cases.py"), "--asan" if asan else "--plain", json.dumps(cases)]
    p = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout, env=env)
    return p.returncode, p.stdout, p.stderr


def _inputs(c, lengths, csr, seed, dtype):
    from sglang_decode import workloads as W
    from oracle import attention as OA
    if csr:
        q, k, v, indptr, indices = W.make_csr_inputs(c, lengths, seed=seed, dtype=dtype, device="cpu")
        return (q, k, v, indices, indptr), lambda scale: OA.csr_attention(q, k, v, indptr, indices, lengths,
                                                                           scale=scale)
    q, k, v, pages = W.make_inputs(c, lengths, seed=seed, dtype=dtype, device="cpu")
    return (q, k, v, pages, None), lambda scale: OA.paged_attention(q, k, v, pages, lengths, c.page_size,
                                                                     scale=scale)


def _check(emu, c, lengths, splits, inputs, expected, mode, kernel, scale, dtype_name, tag):
    import numpy as np
    import types
    import driver as D
    from oracle import plan as OP
    r = D.decode(emu, c, lengths, splits, *inputs, mode=mode, kernel=kernel, scale=scale)
    n = len(lengths)
    o, e = r["out"][:n], expected[:n]
    ns = types.SimpleNamespace(batch_capacity=c.batch_capacity, max_splits=c.max_splits,
                               max_context=c.max_context, workers=c.workers, kv_heads=c.kv_heads,
                               block_kv=c.block_kv)
    ref = OP.full_plan(lengths, splits, n, ns, force=mode)
    p = r["plan"]
    plan_ok = (p["error"] == ref["error"] and p["record_count"] == ref["record_count"]
               and p["counts"][:c.batch_capacity] == ref["counts"] and p["mode"] == ref["mode"]
               and p["num_packs"] == ref["num_packs"])
    if plan_ok and "request" in ref:
        m = ref["record_count"]
        plan_ok = all(p[k][:m] == ref[k][:m] for k in ("request", "split", "begin", "end", "weight"))
        plan_ok = plan_ok and p["order"][:m] == ref["order"]
        npk = ref["num_packs"]
        plan_ok = plan_ok and p["pack_first"][:npk] == ref["pack_first"] and p["pack_count"][:npk] == ref[
            "pack_count"]
    if plan_ok and "static_head" in ref:  # STATIC: the per-worker lists, walked
        plan_ok = OP.walk_lists(p["static_head"], p["static_next"]) == OP.walk_lists(ref["static_head"],
                                                                                     ref["static_next"])
    return dict(case=tag, kernel=r["kernel"], mode=int(mode), dtype=dtype_name,
                violations=int((np.abs(o - e) > 2e-2 + 1e-2 * np.abs(e)).sum()),
                nans=int(np.isnan(o).sum()), tail=float(np.abs(r["out"][n:]).sum()),
                plan_ok=bool(plan_ok), counters=r["sync"], max_err=float(np.nan_to_num(np.abs(o - e), nan=9.0).max())
                if o.size else 0.0)


def _lpt_trials(emu, trials, seed):
    """The device STATIC lists (sgd_greedy_lists: round-based LPT) against the oracle's
    sequential argmin LPT on random weights: batches of 0-300 records, 1-8 kv heads,
    1-512 workers; weights uniform in 1..4, in 1..128, mostly 1 with 5% of them 64..200
    (loads far apart, so rounds of a few tasks), or all equal.  Returns the number of
    trials whose walked lists differ."""
    import numpy as np
    import driver as D
    from oracle import plan as OP
    rng = np.random.default_rng(seed)
    bad = []
    for trial in range(trials):
        n = int(rng.integers(0, 300))
        workers = int(rng.choice([1, 2, 3, 7, 16, 40, 108, 256, 512]))
        hkv = int(rng.choice([1, 2, 8]))
        kind = trial % 4
        if kind == 0:
            w = rng.integers(1, 5, n)
        elif kind == 1:
            w = rng.integers(1, 129, n)
        elif kind == 2:
            w = np.where(rng.random(n) < 0.05, rng.integers(64, 200, n), 1)
        else:
            w = np.full(n, int(rng.integers(1, 9)))
        cap = max(n, 1)
        wd = emu.upload(np.asarray(w, np.int32) if n else np.zeros(1, np.int32))
        count, mode = emu.upload(np.array([n], np.int32)), emu.upload(np.array([2], np.int32))
        head, nxt = emu.array((workers,), np.int32, 77), emu.array((cap * hkv,), np.int32, 77)
        emu.check(emu.lib.sgd_greedy_lists(D.ptr(wd), D.ptr(count), D.ptr(mode), D.ptr(head), D.ptr(nxt), hkv,
                                           workers, cap, None), "greedy_lists")
        ref_head, ref_next = OP.greedy_lists([int(x) for x in w], n, 2, hkv, workers, cap * hkv)
        if OP.walk_lists(head.tolist(), nxt.tolist()) != OP.walk_lists(ref_head, ref_next):
            bad.append(dict(trial=trial, records=n, workers=workers, kv_heads=hkv, kind=kind))
    return dict(case="lpt", trials=trials, mismatches=len(bad), first=bad[:3])


def _upstream(emu, lengths, smax, dtype):
    import ctypes
    import numpy as np
    import driver as D
    from oracle import attention as OA
    from sglang_decode import _lib
    from sglang_decode import workloads as W
    from sglang_decode.config import DecodeConfig
    from sglang_decode.planning.reference import split_records
    import torch
    c = DecodeConfig(batch_capacity=len(lengths), max_splits=smax, max_context=max(4096, max(lengths)),
                     query_heads=8, kv_heads=2, page_size=1, workers=8)
    q, k, v, indptr, indices = W.make_csr_inputs(c, lengths, seed=len(lengths), device="cpu", dtype=dtype)
    splits = W.split_hints(lengths, smax)
    b, hq, d = len(lengths), c.query_heads, c.head_dim
    dt = _lib.dtype_code(dtype)
    qd, kd, vd = emu.upload(D.bits16(q)), emu.upload(D.bits16(k)), emu.upload(D.bits16(v))
    ipd = emu.upload(indptr.numpy().astype(np.int32)[:b + 1])
    idd = emu.upload(indices.numpy().astype(np.int32))
    sd = emu.upload(np.array(splits, np.int32))
    slots = emu.array((b, hq, smax, d), np.float32, np.nan)
    slse = emu.array((b, hq, smax), np.float32, np.nan)
    out = emu.array((b, hq, d), np.uint16)
    qs = (ctypes.c_int64 * 3)(*q.stride())
    kvs = (ctypes.c_int64 * 4)(k.stride(0), k.stride(1), v.stride(0), v.stride(1))
    emu.check(emu.lib.sgd_upstream_decode(D.ptr(qd), D.ptr(kd), D.ptr(vd), D.ptr(out), D.ptr(ipd), D.ptr(idd),
                                          D.ptr(slots), D.ptr(slse), D.ptr(sd), b, smax, hq, c.kv_heads, d, qs, kvs,
                                          ctypes.c_float(d ** -0.5), dt, None), "upstream_decode")
    got = D.from_bits16(out, dt).reshape(out.shape)
    exp = OA.csr_attention(q, k, v, indptr, indices, lengths)[:b]
    viol = int((np.abs(got - exp) > 2e-2 + 1e-2 * np.abs(exp)).sum())
    records, _, _ = split_records(lengths, splits, c)
    table = torch.zeros((b, max(max(lengths), 1)), dtype=torch.int32)
    for r, n in enumerate(lengths):
        table[r, :n] = indices[int(indptr[r]):int(indptr[r]) + n]
    ref = OA.split_partials(q, k[:, None], v[:, None], table, lengths, 1,
                            [(x.request, x.split, x.begin, x.end) for x in records], hq, smax)
    slot_viol = 0
    for (r, h, s), (p, l) in ref.items():
        slot_viol += int((np.abs(slots[r, h, s] - p) > 2e-2 + 1e-2 * np.abs(p)).sum())
        slot_viol += int(abs(slse[r, h, s] - l) > 1e-2 + 1e-3 * abs(l))
    return dict(case="upstream", lengths=lengths, smax=smax, dtype=str(dtype), violations=viol,
                slot_violations=slot_viol, slots=len(ref), nans=int(np.isnan(got).sum()))


def _noalloc(emu, name, batches, mode, dtype):
    import ctypes
    import numpy as np
    import driver as D
    from oracle import attention as OA
    from sglang_decode import _lib
    from sglang_decode import workloads as W
    c = W.config_for(name, workers=64)
    full = W.lengths_for(name)
    out = emu.array((c.batch_capacity, c.query_heads, c.head_dim), np.uint16, 0x7fc0)
    rows = []
    for n, shrink in batches:
        lengths = [max(1, x // shrink) for x in full[:n]]
        splits = W.split_hints(lengths, c.max_splits)
        csr = c.page_size == 1
        inputs, oracle = _inputs(c, lengths, csr, 70 + n, dtype)
        q, k, v, pages, indptr = inputs
        ref = D.decode(emu, c, lengths, splits, q, k, v, pages, indptr, mode=mode)
        L = emu.array((c.batch_capacity,), np.int32, 0)
        S = emu.array((c.batch_capacity,), np.int32, 1)
        L[:n], S[:n] = lengths, splits
        A = emu.upload(np.array([n], np.int32))
        qd, kd, vd = emu.upload(D.bits16(q)), emu.upload(D.bits16(k)), emu.upload(D.bits16(v))
        pd = emu.upload(pages.numpy().astype(np.int32))
        ipd = emu.upload(indptr.numpy().astype(np.int32)) if csr else None
        a = _lib.NoAllocArgsC()
        a.q, a.k, a.v, a.pages = qd.ctypes.data, kd.ctypes.data, vd.ctypes.data, pd.ctypes.data
        a.indptr = ipd.ctypes.data if csr else None
        a.lengths, a.splits, a.active, a.out = L.ctypes.data, S.ctypes.data, A.ctypes.data, out.ctypes.data
        a.scale = float(c.head_dim ** -0.5)
        a.q_stride[:] = list(q.stride())
        if csr:
            a.k_stride[:] = [k.stride(0), 0, k.stride(1), k.stride(2)]
            a.v_stride[:] = [v.stride(0), 0, v.stride(1), v.stride(2)]
            a.pt_stride[:] = [0, 0]
        else:
            a.k_stride[:], a.v_stride[:], a.pt_stride[:] = list(k.stride()), list(v.stride()), list(pages.stride())
        a.batch_capacity, a.max_splits, a.max_context = c.batch_capacity, c.max_splits, c.max_context
        a.query_heads, a.kv_heads, a.head_dim = c.query_heads, c.kv_heads, c.head_dim
        a.page_size, a.csr, a.dtype, a.workers = c.page_size, int(csr), _lib.dtype_code(dtype), c.workers
        a.force_mode, a.kernel = int(mode), _lib.KERNELS["auto"]
        emu.check(emu.lib.sgd_decode_noalloc(ctypes.byref(a), None), "decode_noalloc")
        got = D.from_bits16(out, a.dtype).reshape(out.shape)
        exp = oracle(None)[:n]
        rows.append(dict(batch=n, bitwise=bool(np.array_equal(got, ref["out"], equal_nan=True)),
                         violations=int((np.abs(got[:n] - exp) > 2e-2 + 1e-2 * np.abs(exp)).sum()),
                         tail=float(np.abs(got[n:]).sum())))
    return dict(case="noalloc", workload=name, mode=int(mode), calls=rows)


def _merge_min(emu, bcap, hq, smax, d, min_splits):
    """sgd_merge_splits_min against sgd_merge_splits on synthetic split slots: rows of
    1 <= n < min_splits untouched, every other row bitwise equal, a plan error NaN
    everywhere.  The executor reports one workgroup per CU as resident, so batches of more
    rows than CUs stride."""
    import ctypes
    import numpy as np
    import driver as D
    from sglang_decode import _lib
    rng = np.random.default_rng(5)
    counts = emu.upload(np.array([(0, 1, 2, 16, 17, 64, 1, 3)[r % 8] % (smax + 1) for r in range(bcap)], np.int32))
    partial = emu.upload(rng.standard_normal((bcap, hq, smax, d)).astype(np.float32))
    lse = emu.upload((rng.standard_normal((bcap, hq, smax)) * 3).astype(np.float32))
    active = emu.upload(np.array([bcap], np.int32))
    res = {}
    for tag, m, error in (("full", None, 0), ("min", min_splits, 0), ("error", min_splits, 1)):
        out = emu.array((bcap, hq, d), np.uint16, 0x40e0)  # 7.0 in bf16
        err = emu.upload(np.array([error], np.int32))
        args = (D.ptr(partial), D.ptr(lse), D.ptr(counts), D.ptr(active), D.ptr(err), D.ptr(out), bcap, hq, d, smax)
        if m is None:
            emu.check(emu.lib.sgd_merge_splits(*args, _lib.SGD_BF16, None), "merge_splits")
        else:
            emu.check(emu.lib.sgd_merge_splits_min(*args, m, _lib.SGD_BF16, None), "merge_splits_min")
        res[tag] = np.array(out)
    n = np.array(counts)
    skip = (n >= 1) & (n < min_splits)
    return dict(case="merge_min", rows=bcap * hq, min_splits=min_splits,
                merged_equal=bool(np.array_equal(res["min"][~skip], res["full"][~skip])),
                skipped_untouched=bool((res["min"][skip] == 0x40e0).all()),
                error_nan=bool(np.isnan(D.from_bits16(res["error"], _lib.SGD_BF16)).all()))


def run(cases, asan):
    import torch
    import driver as D
    sys.path.insert(0, TESTS)
    emu = D.Emu(asan=asan)
    for case in cases:
        if "lpt" in case:
            print(json.dumps(_lpt_trials(emu, int(case["lpt"]), int(case.get("seed", 0)))), flush=True)
        elif "upstream" in case:
            lengths, smax = case["upstream"]
            print(json.dumps(_upstream(emu, list(lengths), int(smax), getattr(torch, case.get("dtype", "bfloat16")))),
                  flush=True)
        elif "merge_min" in case:
            bcap, hq, smax, d, m = case["merge_min"]
            print(json.dumps(_merge_min(emu, int(bcap), int(hq), int(smax), int(d), int(m))), flush=True)
        elif "noalloc" in case:
            print(json.dumps(_noalloc(emu, case["noalloc"], case["batches"], int(case.get("mode", -1)),
                                      getattr(torch, case.get("dtype", "bfloat16")))), flush=True)
        elif "sweep" in case:
            from test_gpu_sweep import draw, kernels_for
            seed = int(case["sweep"])
            c, csr, lengths, splits, dtype, mode, scale = draw(seed)
            inputs, oracle = _inputs(c, lengths, csr, seed, dtype)
            expected = oracle(scale)
            for kernel in case.get("kernels") or kernels_for(c, csr):
                print(json.dumps(_check(emu, c, lengths, splits, inputs, expected, int(mode), kernel, scale,
                                        str(dtype), f"sweep {seed}")), flush=True)
        else:
            from sglang_decode import workloads as W
            name = case["workload"]
            c = W.config_for(name, workers=case.get("workers", 256))
            lengths = W.lengths_for(name)[:case.get("requests")]
            splits = W.split_hints(lengths, c.max_splits)
            dtype = getattr(torch, case.get("dtype", "bfloat16"))
            inputs, oracle = _inputs(c, lengths, c.page_size == 1, case.get("seed", 7), dtype)
            expected = oracle(None)
            for kernel in case.get("kernels", ["auto"]):
                for mode in case.get("modes", [-1]):
                    print(json.dumps(_check(emu, c, lengths, splits, inputs, expected, mode, kernel, None,
                                            str(dtype), name)), flush=True)


if __name__ == "__main__":
    sys.path.insert(0, HERE)
    for p in (os.path.join(ROOT, "-sglang-decode-_amd"), ROOT):
        sys.path.insert(0, p)
    run(json.loads(sys.argv[2]), asan=sys.argv[1] == "--asan")
