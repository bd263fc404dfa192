"""Decode-attention benchmark: Llama-3-8B GQA layer, batch 64, on one MI355X.

Workload (the headline configuration, `--workload c2`): batch 64, 32 q heads / 8 kv
heads, head_dim 128, bf16 KV ~ N(0,1), page_size 1 CSR token indices, contexts
clip(round(exp(N(ln 1024, 0.8))), 128, 8192) (seeded), a 1M-token KV pool per layer
with randomly permuted slots.  A step is one hipGraph replay of the plan build plus
the model's layers (persistent attention, merge): 32 for the 8B shapes, 80 for
Llama-3-70B (`--layers` overrides), so the plan -- built once per step and shared by
every layer, as in a decode step -- is counted once per step.  The layers rotate
over a few KV pools of their own (4 x 1M tokens = 16 GB for c2), so every layer's
rows come from HBM: the working set far exceeds the 256 MB Infinity Cache.
`--workload c3` is the skewed batch (2 x 32768 + 126 short requests, up to 64
splits), `--workload c4` the Llama-3-70B paged layer (page 16, 64 q / 8 kv, batch
32, contexts in [2048, 16384], 200k-page pools; `--dtype fp16|bf16`), `--workload
c5` the 32-layer step of the 8B shape at batch 64 (contexts lognormal, median 2048)
with a 256k-token pool per layer.

Reported per schedule (R1, STATIC, STATIC_HOST, D1, D4, R0, AUTO), timed in 5 alternating
rounds as the reference's benchmark does (benchmarks/bench_decode.py:76-91): us/layer =
replay time / layers, achieved GB/s = algorithmic bytes per layer / us/layer, and an
oracle check (layer 0 within 2e-2 abs / 1e-2 rel of the FP32 oracle, and every layer that
reads the same pool bitwise equal to it).  STATIC builds its LPT lists on the device
inside the replay (the reference's device greedy, a serial chain); STATIC_HOST is the
reference benchmark's host-static variant (benchmarks/bench_decode.py:14-30): C++ heap
LPT on the host when the lengths change, uploaded from pinned memory, installed after
the device R1 plan.  AUTO is the adapter's default: no forced mode, the policy artifact
shipped for this GPU (planning.policy.shipped_policy; R1 where none ships) choosing on the
device plan; `default_schedule` names the artifact and the mode its rules picked.
`value` is the achieved HBM GB/s of the fastest schedule.
`roofline` times the attention kernel alone for that schedule: a HIP graph of
back-to-back launches (rotating layers) replayed between HIP events on its stream.
`roofline.traffic` is the HBM bytes per attention launch from two rocprofv3 --pmc passes
(FETCH_SIZE, then WRITE_SIZE) run by this bench in child processes over the same workload,
each scaled by the counter's reading for a copy kernel of known size in the same pass
(`--traffic file` or a failed pass: the committed profiles' lookup, named in
`traffic_source`).
`attention_merge_us` (attention + merge per layer, no plan) and `single_layer_entry_us`
(one layer's full entry: plan build + attention + merge) are timed the same way for that
schedule; `entry` times that full entry per schedule at the reference's own boundary:
eager calls, GPU time and host wall time per call, STATIC_HOST re-planning on the host
and uploading on every call.  `cpu_baseline` is the FP32 oracle on the same inputs on
every host core, and the CPU planning spec, timed on this host (1 warmup, median of 5).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--layers L] [--workload c2]
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "-sglang-decode-_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "decode-attn µs/layer + achieved HBM GB/s (% peak), Llama-3-8B GQA shape B=64"
PEAK_HBM_GBS = 8000.0
POLICIES = ("R1", "STATIC", "STATIC_HOST", "D1", "D4", "R0", "AUTO")
WORKLOADS = {
    "c2": "llama3-8b decode layer: B=64, 32q/8kv, D=128, bf16, CSR page 1, lognormal(median 1024) "
          "contexts clipped [128,8192], 1M-token pool per layer",
    "c3": "skewed decode layer: B=128 (2 x 32768 + 126 x U[32,512]), 32q/8kv, D=128, bf16, CSR page 1, "
          "splits of up to 512 tokens (max 64), 1M-token pool per layer",
    "c4": "llama3-70b paged decode layer: B=32, 64q/8kv, D=128, page 16, contexts U[2048,16384], "
          "200k-page pool per layer",
    "c5": "llama3-8b 32-layer decode step: B=64, 32q/8kv, D=128, bf16, CSR page 1, lognormal(median "
          "2048) contexts clipped [128,16384], 256k-token pool per layer",
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=0,
                    help="layers per step; 0 = the model's: 32 (c2, c3, c5) or 80 (c4)")
    ap.add_argument("--workload", default="c2", choices=sorted(WORKLOADS))
    ap.add_argument("--dtype", default="bf16", choices=("bf16", "fp16"))
    ap.add_argument("--policies", default=",".join(POLICIES))
    ap.add_argument("--kernel", default="auto")
    ap.add_argument("--workers", type=int, default=0, help="0 = default_workers (2 per CU)")
    ap.add_argument("--kernel-launches", type=int, default=200,
                    help="attention-only launches timed for the roofline")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-check", action="store_true")
    ap.add_argument("--json-out", default="")
    ap.add_argument("--kv-store", action="store_true",
                    help="also time the decode step's KV-pool write + q staging: one launch "
                         "(kernels/kv_store.py) against upstream's two scatters and a copy")
    ap.add_argument("--rounds", type=int, default=5,
                    help="alternating timed rounds per schedule (median reported)")
    ap.add_argument("--entry-iterations", type=int, default=200,
                    help="eager single-layer full-entry calls per round and schedule (the reference "
                         "benchmark's boundary, STATIC_HOST planning on the host every call); 0 skips")
    ap.add_argument("--samples-csv", default="",
                    help="write one row per schedule and round (variant, trial, iterations, gpu_us, wall_us, "
                         "status: per step of all layers) for planning.calibrate")
    ap.add_argument("--plan-inputs", action="store_true",
                    help="also time the plan build reading kv_indptr / num_kv_splits itself against the "
                         "reference adapter's copies before it")
    ap.add_argument("--no-upstream", action="store_true",
                    help="skip the upstream two-stage split-KV comparator leg (CSR workloads, groups <= 4)")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="also run a plain N-MiB read+write kernel 5 times, so a rocprofv3 --pmc "
                         "FETCH_SIZE / WRITE_SIZE pass can scale its counts to bytes")
    ap.add_argument("--head-dim", type=int, default=0, choices=(0, 64, 128, 256),
                    help="override the workload's head_dim (0 = its own, 128): the same batch, heads and "
                         "contexts at head_dim 64 or 256")
    ap.add_argument("--no-reference-b", action="store_true",
                    help="skip the reference's published workload B (eager single-layer entries per schedule)")
    ap.add_argument("--traffic-file", default=os.path.join(ROOT, "profiles", "traffic_persistent_decode.json"),
                    help="measured HBM bytes per attention launch (from rocprofv3 --pmc), used for "
                         "roofline.traffic when kernel, schedule and workers match this run")
    ap.add_argument("--traffic", default="live", choices=("live", "file", "off"),
                    help="roofline.traffic: live = two rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE) over "
                         "the reported schedule's attention launches in child processes, scaled by a copy "
                         "kernel in the same passes (falls back to --traffic-file if rocprofv3 fails); "
                         "file = the --traffic-file lookup only")
    ap.add_argument("--traffic-child", action="store_true", help=argparse.SUPPRESS)
    return ap.parse_args()


COPY_MIB = 256


def traffic_child(args):
    """The workload of one live traffic pass (run under rocprofv3 --pmc by the parent): the
    reported schedule's attention launches on one KV pool, then a plain copy kernel of
    COPY_MIB MiB read + written 5 times, whose counts give the counter's bytes scale."""
    import torch
    from sglang_decode import workloads as W
    from sglang_decode.config import Mode
    from sglang_decode.kernels.attention import checked_layout, persistent_decode
    from sglang_decode.runtime.engine import DecodeEngine
    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    dtype = torch.bfloat16 if args.dtype == "bf16" else torch.float16
    c = W.config_for(args.workload, workers=args.workers)
    if args.head_dim:
        import dataclasses
        c = dataclasses.replace(c, head_dim=args.head_dim)
    lengths = W.lengths_for(args.workload)
    splits = W.split_hints(lengths, c.max_splits)
    csr = c.page_size == 1
    if csr:
        x = W.make_csr_inputs(c, lengths, seed=1000, device=dev, dtype=dtype, device_pool=True,
                              pool_tokens=1 << (18 if args.workload == "c5" else 20))
        inputs, indptr = (x[0], x[1], x[2], x[4]), x[3]
    else:
        x = W.make_inputs(c, lengths, seed=1000, device=dev, dtype=dtype, pool_pages=200_000, device_pool=True)
        inputs, indptr = x, None
    engine = DecodeEngine(c, device=dev, dtype=dtype, force_mode=int(Mode[args.policies]), kernel=args.kernel)
    W.update_plan(engine, lengths, splits)
    engine.prepare()
    ks, vs, pts, _ = checked_layout(c, *inputs, indptr, dtype)
    for _ in range(5):
        persistent_decode(engine.plan, engine.layers[0], *inputs, indptr, c.head_dim ** -0.5, ks, vs, pts, csr,
                          args.kernel)
    a = torch.empty(COPY_MIB << 19, dtype=torch.bfloat16, device=dev).fill_(1.0)
    b = torch.empty_like(a)
    for _ in range(5):
        torch.mul(a, 1, out=b)
    torch.cuda.synchronize()


def live_traffic(args, schedule, workers):
    """HBM bytes per attention launch of this run's workload and schedule from two rocprofv3
    --pmc passes (FETCH_SIZE, WRITE_SIZE) over traffic_child, each scaled by what the same
    counter reads for the copy kernel of known size; None if rocprofv3 is missing or a pass
    yields no counts (bounded by a time limit, its process group killed on expiry)."""
    import csv
    import shutil
    import signal
    import subprocess
    import tempfile
    tool = shutil.which("rocprofv3")
    profiled = any(k.startswith("ROCPROF") for k in os.environ) or "rocprof" in os.environ.get("LD_PRELOAD", "")
    if tool is None or profiled:  # no profiler, or this run is itself under one
        return None
    child = [sys.executable, os.path.abspath(__file__), "--traffic-child", "--workload", args.workload,
             "--dtype", args.dtype, "--kernel", args.kernel, "--policies", schedule, "--workers", str(workers),
             "--head-dim", str(args.head_dim)]
    env = dict(os.environ, TMPDIR="/tmp")
    counts = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        out = tempfile.mkdtemp(prefix="sgd_pmc_", dir="/tmp")
        cmd = [tool, "--pmc", counter, "-d", out, "-o", "run", "--output-format", "csv", "--", *child]
        proc = subprocess.Popen(cmd, cwd="/tmp", env=env, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL,
                                start_new_session=True)
        try:
            proc.wait(timeout=240)
        except subprocess.TimeoutExpired:
            os.killpg(proc.pid, signal.SIGKILL)
            proc.wait()
        attn, copy = [], []
        for root, _, files in os.walk(out):
            for name in files:
                if not name.endswith("counter_collection.csv"):
                    continue
                with open(os.path.join(root, name), newline="") as f:
                    for row in csv.DictReader(f):
                        kernel = row.get("Kernel_Name", "")
                        if "k_attention_" in kernel:
                            attn.append(float(row["Counter_Value"]))
                        elif "MulFunctor" in kernel:
                            copy.append(float(row["Counter_Value"]))
        shutil.rmtree(out, ignore_errors=True)
        if not attn or not copy:  # the profiler's own exit code is not trusted either way
            return None
        factor = (sum(copy) / len(copy)) * 1024.0 / (COPY_MIB << 20)
        counts[counter] = (sum(attn) / len(attn)) * 1024.0 / factor, factor
    read, fetch_factor = counts["FETCH_SIZE"]
    written, write_factor = counts["WRITE_SIZE"]
    return dict(read_bytes=round(read), write_bytes=round(written), traffic_bytes=round(read + written),
                fetch_factor=round(fetch_factor, 5), write_factor=round(write_factor, 5))


def measured_traffic(path, kernel, workers, algorithmic_bytes):
    """HBM bytes per launch recorded from rocprofv3 FETCH_SIZE/WRITE_SIZE passes for this
    kernel, worker count and workload (same algorithmic bytes), or None.  The schedule only
    changes which worker reads which rows, not the bytes, so it is not part of the key."""
    try:
        with open(path) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    for row in rec.get("launches", []):
        if (row.get("kernel"), row.get("workers"), row.get("algorithmic_bytes")) == (
                kernel, workers, algorithmic_bytes):
            return row.get("traffic_bytes")
    return None


def graph_time(fn, reps, dev, rounds=5):
    """Median per-call time (us) of fn(0) .. fn(reps - 1) captured in one HIP graph and
    replayed between HIP events on the current stream."""
    import torch
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for i in range(min(reps, 3)):
            fn(i)
    torch.cuda.synchronize()
    cg = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(cg, stream=side):
            for i in range(reps):
                fn(i)
    torch.cuda.synchronize()
    cg.replay()
    durs = []
    for _ in range(rounds):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        cg.replay()
        b.record()
        b.synchronize()
        durs.append(a.elapsed_time(b) * 1000.0 / reps)
    return statistics.median(durs)


def time_kv_store(c, fx, graph, batch, layers, csr, dtype, dev, reps=32, rounds=5):
    """The decode step's KV-pool write + q staging for `batch` new tokens, per layer: one
    launch of kernels/kv_store.py against what the reference adapter runs
    (integrations/sglang_backend.py:91-92, 102-103: set_kv_buffer's two index_put
    scatters, then qbuf[:batch].copy_).  Each captured in a HIP graph of `reps` layers
    (rotating layers), replayed between HIP events; median of `rounds`.  Runs after the
    measured steps: it overwrites `batch` slots of the pools."""
    import torch
    from sglang_decode.kernels.kv_store import store_kv_and_stage_q
    g = torch.Generator(device=dev).manual_seed(99)
    q = torch.randn((batch, c.query_heads, c.head_dim), generator=g, device=dev).to(dtype)
    k = torch.randn((batch, c.kv_heads, c.head_dim), generator=g, device=dev).to(dtype)
    v = torch.randn((batch, c.kv_heads, c.head_dim), generator=g, device=dev).to(dtype)
    caches = []
    for li in range(layers):
        kc, vc = fx[li][1], fx[li][2]
        if not csr:  # paged pools [pages, page, Hkv, D] hold tokens [pages * page, Hkv, D]
            kc, vc = kc.view(-1, c.kv_heads, c.head_dim), vc.view(-1, c.kv_heads, c.head_dim)
        caches.append((kc, vc))
    tokens = caches[0][0].shape[0]
    loc = torch.randperm(tokens, generator=torch.Generator().manual_seed(98))[:batch].to(dev)

    def fused(i):
        kc, vc = caches[i % layers]
        store_kv_and_stage_q(k, v, loc, kc, vc, q, graph.q[i % layers])

    def separate(i):
        kc, vc = caches[i % layers]
        kc[loc] = k
        vc[loc] = v
        graph.q[i % layers][:batch].copy_(q)

    out = {name: round(graph_time(fn, reps, dev, rounds), 2) for name, fn in (("fused_us", fused),
                                                                              ("separate_us", separate))}
    out["tokens"] = batch
    return out


def time_plan_inputs(c, lengths, splits, dev, reps=32, rounds=5):
    """The per-step plan build from the step's CSR metadata: what the reference adapter
    runs (integrations/sglang_backend.py:50-55, 98-99: the active fill, lengths as
    kv_indptr differences, the num_kv_splits copy, then the plan launch) against the one
    launch that reads kv_indptr / num_kv_splits itself (sgd_build_plan_csr).  Each
    captured in a HIP graph of `reps` builds, replayed between HIP events; median."""
    import torch
    from sglang_decode.planning.builder import build_plan
    from sglang_decode.runtime.workspace import PlanBuffers
    plan = PlanBuffers(c, dev)
    sync = torch.zeros(2, dtype=torch.int32, device=dev)
    b = len(lengths)
    indptr = torch.zeros(b + 1, dtype=torch.int32)
    indptr[1:] = torch.cumsum(torch.tensor(lengths, dtype=torch.int64), 0).to(torch.int32)
    indptr = indptr.to(dev)
    num = torch.tensor(splits, dtype=torch.int32, device=dev)

    def copies(_):
        plan.active.fill_(b)
        plan.lengths[:b].copy_(indptr[1:b + 1] - indptr[:b])
        plan.splits[:b].copy_(num[:b])
        build_plan(plan, -1, counters=sync)

    def fused(_):
        build_plan(plan, -1, counters=sync, csr_metadata=(indptr, num, b))

    # From the request pool: kv_indptr / kv_indices / split counts and the plan's inputs in
    # one launch (kernels/csr_metadata.py), then the build -- seq_lens to plan in two launches.
    from sglang_decode.kernels.csr_metadata import csr_metadata
    gen = torch.Generator().manual_seed(97)
    req_to_token = torch.randint(0, 1 << 20, (b, max(lengths)), generator=gen, dtype=torch.int32).to(dev)
    seq_lens = torch.tensor(lengths, dtype=torch.int64, device=dev)
    pool_idx = torch.randperm(b, generator=gen).to(dev)
    meta_indptr = torch.zeros(b + 1, dtype=torch.int32, device=dev)
    meta_indices = torch.zeros(sum(lengths), dtype=torch.int32, device=dev)
    meta_splits = torch.zeros(b, dtype=torch.int32, device=dev)

    def from_pool(_):
        csr_metadata(seq_lens, pool_idx, req_to_token, c.max_splits, meta_indptr, meta_indices, meta_splits,
                     plan=plan)
        build_plan(plan, -1, counters=sync)

    def metadata_only(_):
        csr_metadata(seq_lens, pool_idx, req_to_token, c.max_splits, meta_indptr, meta_indices, meta_splits,
                     plan=plan)

    out = {name: round(graph_time(fn, reps, dev, rounds), 2) for name, fn in (
        ("fused_us", fused), ("copies_us", copies), ("from_pool_us", from_pool), ("metadata_us", metadata_only))}
    out["batch"] = b
    out["tokens"] = sum(lengths)
    return out


# The reference's one published workload (benchmarks/workloads.py:7, workload B) and its
# figure, taken from the author's earlier materials on unstated hardware (A100 inferred from
# configs/a100_bf16.json) and not re-measured there (docs/resume_mapping.md:26).
REFERENCE_B = [256] * 24 + [1536] * 4 + [16384] * 4
REFERENCE_B_PUBLISHED = dict(R0_us=237.0, D4_us=214.0, hardware="not stated (A100 inferred)",
                             source="docs/resume_mapping.md:26",
                             note="history from other hardware, not re-measured by the reference; not a target")


def time_reference_workload_b(dev, dtype, worker_counts, iterations, rounds, threads):
    """Workload B at the reference's own boundary (benchmarks/bench_decode.py:33-97): the
    default DecodeConfig (page 16, 32 q / 8 kv heads, head_dim 128, batch capacity 64),
    split hints, the reference's input generator (seed 17, a pool of exactly the used
    pages), one layer called eagerly -- plan build + attention + merge per call -- per
    schedule, STATIC_CPU planning its lists on the host every call.  Alternating rounds of
    `iterations` calls; GPU time per call from HIP events and host wall time per call,
    medians.  Each schedule's output is checked against the FP32 oracle."""
    import numpy as np
    import torch
    from oracle import attention as OA
    from sglang_decode import workloads as W
    from sglang_decode.config import DecodeConfig, Mode
    from sglang_decode.planning.host_static import HostStatic
    from sglang_decode.runtime.engine import DecodeEngine
    lengths = REFERENCE_B
    b = len(lengths)
    per_workers, check = {}, {}
    for workers in worker_counts:
        c = DecodeConfig(workers=workers)
        splits = W.split_hints(lengths, c.max_splits)
        q, k, v, table = W.make_inputs(c, lengths, seed=17, device=dev, dtype=dtype)
        if not check:
            expected = OA.paged_attention_threads(q[:b].cpu(), k.cpu(), v.cpu(), table[:b].cpu(), lengths,
                                                  c.page_size, threads=threads)[:b]
        calls = {}
        for name in ("R0", "R1", "STATIC", "STATIC_CPU", "D1", "D4"):
            mode = Mode.R1 if name == "STATIC_CPU" else Mode[name]
            eng = DecodeEngine(c, device=dev, dtype=dtype, force_mode=int(mode))
            W.update_plan(eng, lengths, splits)
            if name == "STATIC_CPU":
                hs = HostStatic(eng)

                def call(eng=eng, hs=hs):
                    hs.plan_lists(lengths, splits)
                    eng.prepare()
                    hs.apply()
                    return eng.execute(q, k, v, table)
            else:
                def call(eng=eng):
                    eng.prepare()
                    return eng.execute(q, k, v, table)
            out = call()
            torch.cuda.synchronize()
            got = out[:b].float().cpu().numpy()
            ok = bool(np.allclose(got, expected, atol=2e-2, rtol=1e-2))
            prev = check.get(name)
            check[name] = dict(ok=ok and (prev is None or prev["ok"]),
                               max_abs_err=round(float(np.max(np.abs(got - expected))), 6))
            for _ in range(max(1, iterations // 10)):
                call()
            calls[name] = call
        torch.cuda.synchronize()
        rows = {name: ([], []) for name in calls}
        for trial in range(rounds):
            for name in (list(calls) if trial % 2 == 0 else list(reversed(calls))):
                start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                torch.cuda.synchronize()
                wall0 = time.perf_counter_ns()
                start.record()
                for _ in range(iterations):
                    calls[name]()
                end.record()
                end.synchronize()
                rows[name][0].append(start.elapsed_time(end) * 1000.0 / iterations)
                rows[name][1].append((time.perf_counter_ns() - wall0) / 1000.0 / iterations)
        per_workers[str(workers)] = {name: dict(gpu_us=round(statistics.median(g), 2),
                                                wall_us=round(statistics.median(w), 2)) for name, (g, w) in rows.items()}
    dt = "bf16" if dtype == torch.bfloat16 else "fp16"
    return dict(lengths="[256]*24 + [1536]*4 + [16384]*4",
                config=f"DecodeConfig() defaults: batch capacity 64, 32q/8kv, D=128, page 16, max_splits 16, "
                       f"split_hints; {dt}",
                boundary="eager single-layer full entry (plan + attention + merge) per call",
                iterations=iterations, rounds=rounds, workers=per_workers, check=check,
                published=REFERENCE_B_PUBLISHED)


def provenance(dev, args, config, lengths, splits):
    """What produced this line: a hash of the sources that build and drive the path, the
    software versions, the device, and a hash of the workload (benchmarks/common.py:12-30 of
    the reference writes the same kind of manifest)."""
    import hashlib
    import platform
    import subprocess
    import torch
    h = hashlib.sha256()
    for base, exts in ((os.path.join(ROOT, "-sglang-decode-_amd"), (".hip", ".h", ".py")),
                       (os.path.join(ROOT, "include"), (".h",))):
        for dirpath, dirnames, files in sorted(os.walk(base)):
            dirnames[:] = sorted(d for d in dirnames if not d.startswith(("_", ".")))
            for f in sorted(files):
                if f.endswith(exts):
                    h.update(f.encode())
                    with open(os.path.join(dirpath, f), "rb") as fh:
                        h.update(fh.read())
    with open(os.path.abspath(__file__), "rb") as fh:
        h.update(fh.read())
    try:
        git = subprocess.run(["git", "rev-parse", "HEAD"], cwd=ROOT, capture_output=True, text=True,
                             timeout=10).stdout.strip() or None
    except (OSError, subprocess.SubprocessError):
        git = None
    props = torch.cuda.get_device_properties(dev)
    wl = json.dumps(dict(config=repr(config), lengths=list(lengths), splits=list(splits)), sort_keys=True)
    return dict(source_sha256=h.hexdigest()[:16], git=git, torch=torch.__version__, hip=torch.version.hip,
                python=platform.python_version(), device=props.name,
                arch=getattr(props, "gcnArchName", None), compute_units=props.multi_processor_count,
                workload_sha256=hashlib.sha256(wl.encode()).hexdigest()[:16], argv=sys.argv[1:])


def main():
    args = parse()
    if args.traffic_child:
        traffic_child(args)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (the decode path "
              "has no collective; each GPU would run its own share of the batch or of the KV heads)",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from sglang_decode import workloads as W
    from sglang_decode.config import Mode, default_workers
    from sglang_decode.kernels.attention import persistent_decode
    from sglang_decode.runtime.engine import DecodeEngine, PlanKey
    from sglang_decode.runtime.graph import DecodeGraph
    from sglang_decode.planning.host_static import HostStatic
    from sglang_decode.planning.policy import load_policy, shipped_policy

    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    props = torch.cuda.get_device_properties(dev)
    workers = args.workers or default_workers(dev)
    dtype = torch.bfloat16 if args.dtype == "bf16" else torch.float16
    c = W.config_for(args.workload, workers=workers)
    if args.head_dim:
        import dataclasses
        c = dataclasses.replace(c, head_dim=args.head_dim)
    lengths = W.lengths_for(args.workload)
    splits = W.split_hints(lengths, c.max_splits)
    batch = len(lengths)
    layers = args.layers or {"c4": 80}.get(args.workload, 32)
    # distinct KV pools (and q, indices) the layers rotate over; each is used again only
    # after the others' rows have streamed through the caches
    pools = min(layers, {"c4": 2, "c5": 32}.get(args.workload, 4))
    csr = c.page_size == 1
    print(f"[bench] device={props.name} CUs={props.multi_processor_count} workers={workers} "
          f"workload={args.workload} batch={batch} sumL={sum(lengths)} layers={layers} pools={pools}", flush=True)

    if csr:
        pool_tokens = 1 << (18 if args.workload == "c5" else 20)
        fx = [W.make_csr_inputs(c, lengths, seed=1000 + i, device=dev, pool_tokens=pool_tokens, dtype=dtype,
                                device_pool=True) for i in range(pools)]
        fx = [fx[i % pools] for i in range(layers)]
        graph_kw = dict(index_capacity=[x[4].numel() for x in fx])
        tables = [x[4] for x in fx]
    else:
        fx = [W.make_inputs(c, lengths, seed=1000 + i, device=dev, dtype=dtype, pool_pages=200_000,
                            device_pool=True) for i in range(pools)]
        fx = [fx[i % pools] for i in range(layers)]
        graph_kw = {}
        tables = [x[3][:batch] for x in fx]
    bytes_per_layer = W.algorithmic_bytes(lengths, c)
    torch.cuda.synchronize()

    # the oracle's view of pool 0 (the pool of layer 0), gathered to the host once, outside
    # any timed region: the used KV rows or pages, relabelled, with q -- a paged layout
    # for the threaded CPU oracle (CSR rows are pages of one token)
    from oracle import attention as OA
    x = fx[0]
    if csr:
        idx = x[4].long()
        rows_k, rows_v = x[1][idx].cpu()[:, None], x[2][idx].cpu()[:, None]
        table = torch.zeros((batch, max(lengths)), dtype=torch.int32)
        starts = x[3][:batch].cpu().tolist()
        for r, n in enumerate(lengths):
            table[r, :n] = torch.arange(starts[r], starts[r] + n, dtype=torch.int32)
        host = (x[0][:batch].cpu(), rows_k, rows_v, table, 1)
    else:
        used = [x[3][r, :(n + c.page_size - 1) // c.page_size].long() for r, n in enumerate(lengths)]
        flat = torch.cat(used)
        table = torch.full((batch, c.max_pages), -1, dtype=torch.int32)
        cursor = 0
        for r, u in enumerate(used):
            table[r, :u.numel()] = torch.arange(cursor, cursor + u.numel(), dtype=torch.int32)
            cursor += u.numel()
        host = (x[0][:batch].cpu(), x[1][flat].cpu(), x[2][flat].cpu(), table, c.page_size)
    cpu_threads = len(os.sched_getaffinity(0))
    oracle = lambda: OA.paged_attention_threads(*host[:4], lengths, host[4], threads=cpu_threads)[:batch]
    expected = None if args.no_check and args.no_cpu_baseline else oracle()

    engines, hosts, samples = {}, {}, []
    host_lpt_us = None
    auto_policy = shipped_policy(dev)
    for name in [p for p in args.policies.split(",") if p]:
        host_static = name == "STATIC_HOST"
        auto = name == "AUTO"
        mode = -1 if auto else int(Mode.R1 if host_static else Mode[name])
        engine = DecodeEngine(c, device=dev, dtype=dtype, layers=layers, force_mode=mode, kernel=args.kernel,
                              rules=load_policy(auto_policy) if auto else ())
        if host_static:
            # the host lists go into the plan's static_head / static_next, which the R1 build
            # inside the replay leaves alone; the replay then only forces STATIC
            hs = HostStatic(engine)
            hosts[name] = (hs, engine.prepare)
            t0 = time.perf_counter()
            hs.plan_lists(lengths, splits)
            torch.cuda.synchronize()
            host_lpt_us = (time.perf_counter() - t0) * 1e6
            device_prepare = engine.prepare

            def prepare(device_prepare=device_prepare, hs=hs):
                device_prepare()
                hs.apply()
            engine.prepare = prepare
        key = PlanKey(args.workload, "hints", (c.query_heads, c.kv_heads, c.head_dim))
        graph = DecodeGraph(engine, [key] * layers, [(x[1], x[2]) for x in fx], **graph_kw)
        graph.update([x[0][:batch] for x in fx], tables, lengths, splits)
        graph.capture()
        for _ in range(args.warmup):
            graph.replay()
        engines[name] = (engine, graph)
    torch.cuda.synchronize()

    # alternating rounds (benchmarks/bench_decode.py:76-91): the schedules in order on even
    # rounds, reversed on odd ones; per round the mean of `steps` replays.  STATIC_HOST plans
    # its lists on the host and uploads them before every replay, as a decode step whose
    # lengths change every step would (the reference's STATIC_CPU charges the host LPT on
    # every call); wall_us therefore includes the host planning.
    rounds = {name: [] for name in engines}
    for trial in range(args.rounds):
        for name in (list(engines) if trial % 2 == 0 else list(reversed(engines))):
            graph = engines[name][1]
            replan = hosts[name][0].plan_lists if name in hosts else None
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            wall0 = time.perf_counter_ns()
            start.record()
            for _ in range(args.steps):
                if replan is not None:
                    replan(lengths, splits)
                graph.replay()
            end.record()
            end.synchronize()
            rounds[name].append(start.elapsed_time(end) / args.steps)
            # STATIC_HOST is the reference benchmark's STATIC_CPU variant
            samples.append(dict(variant="STATIC_CPU" if name == "STATIC_HOST" else name, trial=trial,
                                iterations=args.steps, gpu_us=round(rounds[name][-1] * 1000.0, 3),
                                wall_us=round((time.perf_counter_ns() - wall0) / 1000.0 / args.steps, 3),
                                status="ok"))
    results = {}
    for name, (engine, graph) in engines.items():
        ms_step = statistics.median(rounds[name])
        us_layer = ms_step * 1000.0 / layers
        results[name] = dict(ms_per_step=ms_step, us_per_layer=us_layer,
                             gbps=bytes_per_layer / (us_layer * 1e-6) / 1e9)
        print(f"[bench] {name}: {us_layer:.2f} us/layer  {results[name]['gbps']:.0f} GB/s "
              f"({100 * results[name]['gbps'] / PEAK_HBM_GBS:.1f}% of peak)", flush=True)

    default_schedule = None
    if "AUTO" in engines:  # the mode the shipped policy's rules picked on the device plan
        picked = Mode(int(engines["AUTO"][0].plan.mode.item())).name
        default_schedule = dict(policy=os.path.relpath(auto_policy, ROOT) if auto_policy else None, mode=picked,
                                us_per_layer=round(results["AUTO"]["us_per_layer"], 2))
        print(f"[bench] AUTO (adapter default): policy {default_schedule['policy']} picked {picked}", flush=True)

    if args.samples_csv:
        import csv
        with open(args.samples_csv, "w", newline="") as f:
            w = csv.DictWriter(f, fieldnames=["variant", "trial", "iterations", "gpu_us", "wall_us", "status"])
            w.writeheader()
            w.writerows(samples)

    # every reported schedule against the FP32 oracle: after one more replay, every layer
    # that reads pool 0 (layers 0, pools, 2 * pools, ...) must equal layer 0 bit for bit,
    # and layer 0 must be within 2e-2 abs / 1e-2 rel of the oracle
    check = None
    if not args.no_check:
        check, failed = {}, []
        for name, (engine, graph) in engines.items():
            graph.replay()
            torch.cuda.synchronize()
            out0 = engine.layers[0].output[:batch]
            same = all(torch.equal(engine.layers[li].output[:batch], out0) for li in range(0, layers, pools))
            out = out0.float().cpu().numpy()
            ok = bool(np.allclose(out, expected, atol=2e-2, rtol=1e-2)) and same
            check[name] = dict(ok=ok, max_abs_err=round(float(np.max(np.abs(out - expected))), 6))
            if not ok:
                failed.append(name)
        print(f"[bench] oracle check: {check}", flush=True)
        if failed:
            print(f"[bench] OUTPUT MISMATCH against the oracle: {failed}", file=sys.stderr)
            sys.exit(3)
    best = min(results, key=lambda k: results[k]["us_per_layer"])
    engine, graph = engines[best]

    # roofline: the attention kernel alone, a batch of launches back to back (rotating
    # layers) captured in a HIP graph and replayed between two HIP events on its stream,
    # so no host work and no other kernel sits between launches (each launch returns its
    # claim counter to zero when its last worker finishes).  The mean per launch over a
    # replay; the median of 5 replays is reported.
    p = engine.plan
    stream = torch.cuda.current_stream(dev)
    engine.prepare()

    def launch(i):
        li = i % layers
        layer = engine.layers[li]
        x = fx[li]
        if csr:
            ks = (x[1].stride(0), 0, x[1].stride(1), x[1].stride(2))
            vs = (x[2].stride(0), 0, x[2].stride(1), x[2].stride(2))
            pts = (0, 0)
        else:
            ks, vs, pts = x[1].stride(), x[2].stride(), graph.pages[li].stride()
        persistent_decode(p, layer, graph.q[li], x[1], x[2], graph.pages[li], graph.indptr[li],
                          c.head_dim ** -0.5, ks, vs, pts, csr, args.kernel)

    for layer in engine.layers:
        layer.counter.zero_()
    for i in range(layers):
        launch(i)
    torch.cuda.synchronize()
    batch_n = max(1, args.kernel_launches // 5)
    side = torch.cuda.Stream(dev)
    side.wait_stream(stream)
    kgraph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(kgraph, stream=side):
            for i in range(batch_n):
                launch(i)
    torch.cuda.synchronize()
    kgraph.replay()
    durs = []
    for _ in range(5):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(stream)
        kgraph.replay()
        end.record(stream)
        end.synchronize()
        durs.append(start.elapsed_time(end) * 1000.0 / batch_n)
    kern_us = statistics.median(durs)
    achieved = bytes_per_layer / (kern_us * 1e-6) / 1e9
    kernel_name = engine.attention_kernel_name()
    # traffic and traffic_source are filled in after every timed leg (live_traffic)
    roofline = dict(bound="hbm", achieved=round(achieved, 1), peak=PEAK_HBM_GBS, unit="GB/s",
                    frac=round(achieved / PEAK_HBM_GBS, 4), traffic=None, traffic_source=None,
                    attention_kernel=kernel_name,
                    kernel="persistent_decode", kernel_us=round(kern_us, 2),
                    algorithmic_bytes=bytes_per_layer)
    print(f"[bench] attention kernel alone ({best}): {kern_us:.2f} us  {achieved:.0f} GB/s", flush=True)

    # the reference's other boundaries (benchmarks/bench_decode.py:94): one layer's full
    # entry (plan build + attention + merge) and attention + merge without the plan, per
    # layer, for the reported schedule
    def layer_call(i):
        li = i % layers
        engine.execute(graph.q[li], *graph.kv_pairs[li], graph.pages[li], layer=li, indptr=graph.indptr[li])

    def full_entry(i):
        engine.prepare()
        layer_call(0)

    attn_merge_us = graph_time(layer_call, layers, dev)
    single_layer_us = graph_time(full_entry, 8, dev)
    print(f"[bench] attention + merge ({best}): {attn_merge_us:.2f} us/layer; single-layer full entry "
          f"(plan + attention + merge): {single_layer_us:.2f} us", flush=True)

    # the reference benchmark's external comparator (benchmarks/baselines.py:8-34): upstream
    # SGLang's two-stage split-KV decode on the same inputs and split counts, per layer over the
    # same rotating pools, captured in a HIP graph like the attention + merge figure
    upstream = None
    if csr and not args.no_upstream and c.group_size <= 4 and c.head_dim == 128:
        from sglang_decode.kernels.upstream import decode_attention_fwd
        num = torch.tensor(splits, dtype=torch.int32, device=dev)
        up_logits = torch.empty((batch, c.query_heads, c.max_splits, c.head_dim), device=dev)
        up_lse = torch.empty((batch, c.query_heads, c.max_splits), device=dev)
        up_out = [torch.empty((batch, c.query_heads, c.head_dim), dtype=dtype, device=dev) for _ in range(pools)]

        def up_call(i):
            x = fx[i % layers]
            decode_attention_fwd(x[0][:batch], x[1], x[2], up_out[i % pools], x[3][:batch + 1], x[4], up_logits, up_lse,
                                 num, c.max_splits, c.head_dim ** -0.5)

        up_us = graph_time(up_call, layers, dev)
        up_check = None
        if expected is not None:
            up_call(0)
            torch.cuda.synchronize()
            got = up_out[0].float().cpu().numpy()
            up_check = dict(ok=bool(np.allclose(got, expected, atol=2e-2, rtol=1e-2)),
                            max_abs_err=round(float(np.max(np.abs(got - expected))), 6))
        upstream = dict(us_per_layer=round(up_us, 2), gbps=round(bytes_per_layer / (up_us * 1e-6) / 1e9, 1),
                        check=up_check, splits=f"split_hints(L, {c.max_splits})")
        print(f"[bench] upstream two-stage split-KV (gfx950 rebuild): {up_us:.2f} us/layer "
              f"({upstream['gbps']:.0f} GB/s), check {up_check}", flush=True)

    plan_inputs = None
    if args.plan_inputs:
        plan_inputs = time_plan_inputs(c, lengths, splits, dev)
        print(f"[bench] plan build per step: reading the CSR metadata {plan_inputs['fused_us']:.2f} us, "
              f"copies + build {plan_inputs['copies_us']:.2f} us; from the request pool (metadata launch "
              f"{plan_inputs['metadata_us']:.2f} us + build) {plan_inputs['from_pool_us']:.2f} us", flush=True)
    kv_store = None
    if args.kv_store:
        kv_store = time_kv_store(c, fx, graph, batch, layers, csr, dtype, dev)
        print(f"[bench] kv write + q staging per layer: one launch {kv_store['fused_us']:.2f} us, "
              f"upstream scatters + copy {kv_store['separate_us']:.2f} us", flush=True)

    if args.copy_calibration_mib:
        # a plain copy kernel of known size: N MiB read + N MiB written per launch
        n = args.copy_calibration_mib * (1 << 20) // 2
        a = torch.randn(n, device=dev).to(torch.bfloat16)
        b = torch.empty_like(a)
        for _ in range(5):
            torch.mul(a, 1, out=b)
        torch.cuda.synchronize()
        print(f"[bench] copy calibration: 5 x {args.copy_calibration_mib} MiB read+write", flush=True)

    # the reference's benchmark boundary (benchmarks/bench_decode.py:44-91): eager single-layer
    # full-entry calls -- plan + attention + merge, STATIC_HOST also planning its LPT lists
    # on the host and uploading them on every call -- in alternating rounds; GPU time from
    # HIP events and host wall time per call, medians over the rounds
    entry = {}
    if args.entry_iterations > 0:
        calls = {}
        for name, (eng, gr) in engines.items():
            def call(name=name, eng=eng, gr=gr):
                if name == "STATIC_HOST":  # host LPT + upload, the R1 build, STATIC forced: once each
                    hs, device_prepare = hosts[name]
                    hs.plan_lists(lengths, splits)
                    device_prepare()
                    hs.apply()
                else:
                    eng.prepare()
                eng.execute(gr.q[0], *gr.kv_pairs[0], gr.pages[0], layer=0, indptr=gr.indptr[0])
            for _ in range(max(1, args.entry_iterations // 10)):
                call()
            calls[name] = call
        torch.cuda.synchronize()
        rows = {name: ([], []) for name in calls}
        for trial in range(args.rounds):
            for name in (list(calls) if trial % 2 == 0 else list(reversed(calls))):
                start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                torch.cuda.synchronize()
                wall0 = time.perf_counter_ns()
                start.record()
                for _ in range(args.entry_iterations):
                    calls[name]()
                end.record()
                end.synchronize()
                rows[name][0].append(start.elapsed_time(end) * 1000.0 / args.entry_iterations)
                rows[name][1].append((time.perf_counter_ns() - wall0) / 1000.0 / args.entry_iterations)
        entry = {name: dict(gpu_us=round(statistics.median(g), 2), wall_us=round(statistics.median(w), 2))
                 for name, (g, w) in rows.items()}
        print(f"[bench] single-layer full entry per call (eager, reference boundary): {entry}", flush=True)

    reference_b = None
    if not args.no_reference_b and args.entry_iterations > 0:
        cus = props.multi_processor_count
        reference_b = time_reference_workload_b(dev, dtype, (cus, 2 * cus), args.entry_iterations, args.rounds,
                                                cpu_threads)
        print(f"[bench] reference workload B (eager full entry per call, us): {reference_b['workers']}; "
              f"check {reference_b['check']}", flush=True)
        if not all(v["ok"] for v in reference_b["check"].values()):
            print("[bench] OUTPUT MISMATCH against the oracle on workload B", file=sys.stderr)
            sys.exit(3)

    cpu = None
    if not args.no_cpu_baseline:
        # the FP32 oracle over the full layer (every request) on every host core, and the CPU
        # planning spec (split_records -> bucket_order -> make_packs -> greedy_static) on the
        # same lengths: 1 warmup, then the median of 5 runs each
        from sglang_decode.planning import reference as R

        def cpu_plan():
            recs, _, _ = R.split_records(lengths, splits, c)
            R.make_packs(recs, R.bucket_order(recs), c.kv_heads, c.workers)
            R.greedy_static(recs, c.kv_heads, c.workers)

        def median_of(fn, runs=5):
            fn()
            times = []
            for _ in range(runs):
                t0 = time.perf_counter()
                fn()
                times.append(time.perf_counter() - t0)
            return statistics.median(times)

        t = median_of(oracle)
        plan_t = median_of(cpu_plan)
        cpu = dict(value=round(t * 1e6, 1), unit="us/layer", cores=cpu_threads, kind="port", runs=5, warmup=1,
                   sample=f"FP32 oracle (reference/attention.py:5-18 restated in torch CPU fp32) over the full "
                          f"layer ({batch} requests, {sum(lengths)} context tokens) on {cpu_threads} host threads, "
                          f"median of 5 after 1 warmup",
                   tokens_per_s=round(batch / t, 2), kv_tokens_per_s=round(sum(lengths) / t, 1),
                   plan_us=round(plan_t * 1e6, 1),
                   plan_sample="CPU planning spec (split_records, bucket_order, make_packs, greedy_static) on the "
                               "same lengths, one thread, median of 5 after 1 warmup")
        print(f"[bench] cpu baseline: {t * 1e3:.1f} ms/layer on {cpu_threads} threads; planning spec "
              f"{plan_t * 1e6:.0f} us", flush=True)

    # the live traffic passes last: their child processes run under the profiler after every
    # timed leg of this run is done
    if args.traffic == "live":
        # the bytes do not depend on the schedule (it only changes which worker reads which
        # rows); schedules that are not a device mode are counted as D1
        live = live_traffic(args, "D1" if best in ("AUTO", "STATIC_HOST") else best, workers)
        if live is not None:
            roofline["traffic"] = live["traffic_bytes"]
            roofline["traffic_source"] = dict(kind="rocprofv3 --pmc in this run", **live)
            print(f"[bench] live HBM traffic per attention launch: {live['read_bytes'] / 1e6:.2f} MB read + "
                  f"{live['write_bytes'] / 1e6:.2f} MB written (FETCH_SIZE scale {live['fetch_factor']})",
                  flush=True)
    if roofline["traffic"] is None and args.traffic != "off":
        roofline["traffic"] = measured_traffic(args.traffic_file, kernel_name, workers, bytes_per_layer)
        if roofline["traffic"] is not None:
            roofline["traffic_source"] = dict(kind="file", path=os.path.relpath(args.traffic_file, ROOT))

    r = results[best]
    line = {
        "metric": METRIC, "value": round(r["gbps"], 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(r["ms_per_step"], 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": args.dtype,
        "data": f"synthetic (seeded contexts, N(0,1) {args.dtype} q/K/V, randomly permuted KV pools)",
        "config": {"workload": WORKLOADS[args.workload], "name": args.workload,
                   "batch": batch, "sum_context": sum(lengths), "layers_per_step": layers, "kv_pools": pools,
                   "schedule": best, "workers": workers, "kernel": args.kernel,
                   "splits_total": sum(splits)},
        "us_per_layer": round(r["us_per_layer"], 2),
        "pct_peak_hbm": round(100 * r["gbps"] / PEAK_HBM_GBS, 2),
        "tokens_per_s": round(batch / (r["us_per_layer"] * 1e-6), 1),
        "kv_tokens_per_s": round(sum(lengths) / (r["us_per_layer"] * 1e-6), 1),
        "schedules": {k: {kk: round(vv, 3) for kk, vv in v.items()} for k, v in results.items()},
        "host_lpt_us": None if host_lpt_us is None else round(host_lpt_us, 1),
        "default_schedule": default_schedule,
        "check": check,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "attention_merge_us": round(attn_merge_us, 2),
        "single_layer_entry_us": round(single_layer_us, 2),
        "entry": entry,
        "upstream_comparator": upstream,
        "reference_workload_B": reference_b,
        "provenance": provenance(dev, args, c, lengths, splits),
    }
    if kv_store is not None:
        line["kv_store"] = kv_store
    if plan_inputs is not None:
        line["plan_inputs"] = plan_inputs
    text = json.dumps(line)
    if args.json_out:
        with open(args.json_out, "w") as f:
            f.write(text + "\n")
    print(text, flush=True)


if __name__ == "__main__":
    main()
