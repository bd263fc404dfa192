"""Decode-attention benchmark: Llama-3-8B GQA layer, batch 64, on one MI355X.

Workload (the headline configuration): batch 64, 32 q heads / 8 kv heads, head_dim
128, bf16 KV ~ N(0,1), page_size 1 CSR token indices, contexts
clip(round(exp(N(ln 1024, 0.8))), 128, 8192) (seeded), a 1M-token KV pool per layer
with randomly permuted slots.  A step is one hipGraph replay of the plan build
plus `--layers` layers (counter reset, persistent attention, merge), each layer
over its own KV pool so the working set exceeds the 256 MB Infinity Cache.

Reported per schedule (R1, STATIC, D1, D4, R0): us/layer = replay time / layers,
achieved GB/s = algorithmic bytes per layer / us/layer.  `value` is the achieved
HBM GB/s of the fastest schedule.  `roofline` times the attention kernel alone
(HIP events on the launch stream around each launch, rotating layers) for that
schedule.  `cpu_baseline` is the FP32 oracle on the same inputs, timed on this
host (bounded sample stated in the record).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--layers L]
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
POLICIES = ("R1", "STATIC", "D1", "D4", "R0")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--policies", default=",".join(POLICIES))
    ap.add_argument("--kernel", default="auto")
    ap.add_argument("--workers", type=int, default=0, help="0 = default_workers (2 per CU)")
    ap.add_argument("--kernel-launches", type=int, default=200,
                    help="attention-only launches timed for the roofline")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-check", action="store_true")
    ap.add_argument("--json-out", default="")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="also run a plain N-MiB read+write kernel 5 times, so a rocprofv3 --pmc "
                         "FETCH_SIZE / WRITE_SIZE pass can scale its counts to bytes")
    ap.add_argument("--traffic-file", default=os.path.join(ROOT, "profiles", "traffic_persistent_decode.json"),
                    help="measured HBM bytes per attention launch (from rocprofv3 --pmc), used for "
                         "roofline.traffic when kernel, schedule and workers match this run")
    return ap.parse_args()


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


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (this path needs "
              "no collective; see DESIGN.md for how it would shard)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from sglang_decode import workloads as W
    from sglang_decode.config import Mode, default_workers
    from sglang_decode.kernels.attention import persistent_decode
    from sglang_decode.runtime.engine import DecodeEngine, PlanKey
    from sglang_decode.runtime.graph import DecodeGraph

    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    props = torch.cuda.get_device_properties(dev)
    workers = args.workers or default_workers(dev)
    base = W.config_for("c2", workers=workers)
    c = base
    lengths = W.c2_lengths()
    splits = W.split_hints(lengths, c.max_splits)
    batch = len(lengths)
    pool_tokens = 1 << 20
    layers = args.layers
    print(f"[bench] device={props.name} CUs={props.multi_processor_count} workers={workers} "
          f"batch={batch} sumL={sum(lengths)} layers={layers}", flush=True)

    fx = [W.make_csr_inputs(c, lengths, seed=1000 + i, device=dev, pool_tokens=pool_tokens,
                            device_pool=True) for i in range(layers)]
    bytes_per_layer = W.algorithmic_bytes(lengths, c)
    torch.cuda.synchronize()

    results = {}
    engines = {}
    for name in [p for p in args.policies.split(",") if p]:
        mode = int(Mode[name])
        engine = DecodeEngine(c, device=dev, layers=layers, force_mode=mode, kernel=args.kernel)
        key = PlanKey("c2", "hints", (c.query_heads, c.kv_heads, c.head_dim))
        graph = DecodeGraph(engine, [key] * layers, [(x[1], x[2]) for x in fx],
                            indptrs=[x[4].numel() for x in fx])
        graph.update([x[0][:batch] for x in fx], [x[4] for x in fx], lengths, splits,
                     [x[3] for x in fx])
        graph.capture()
        for _ in range(args.warmup):
            graph.replay()
        torch.cuda.synchronize()
        rounds = []
        for _ in range(3):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            start.record()
            for _ in range(args.steps):
                graph.replay()
            end.record()
            end.synchronize()
            rounds.append(start.elapsed_time(end) / args.steps)
        ms_step = statistics.median(rounds)
        us_layer = ms_step * 1000.0 / layers
        results[name] = dict(ms_per_step=ms_step, us_per_layer=us_layer,
                             gbps=bytes_per_layer / (us_layer * 1e-6) / 1e9)
        engines[name] = (engine, graph)
        print(f"[bench] {name}: {us_layer:.2f} us/layer  {results[name]['gbps']:.0f} GB/s "
              f"({100 * results[name]['gbps'] / PEAK_HBM_GBS:.1f}% of peak)", flush=True)

    best = min(results, key=lambda k: results[k]["us_per_layer"])
    engine, graph = engines[best]

    # correctness of the reported schedule: layer 0 against the FP32 oracle.  The used KV
    # rows are gathered to the host first (outside any timed region).
    from oracle import attention as OA
    x = fx[0]
    idx = x[4].long()
    host = (x[0].cpu(), x[1][idx].cpu(), x[2][idx].cpu(), x[3].cpu(),
            torch.arange(idx.numel(), dtype=torch.int32))
    check, cpu_times, expected = None, [], None
    if not (args.no_check and args.no_cpu_baseline):
        t0 = time.perf_counter()
        expected = OA.csr_attention(*host, lengths)[:batch]
        cpu_times.append(time.perf_counter() - t0)
    if not args.no_check:
        graph.replay()
        torch.cuda.synchronize()
        out = engine.layers[0].output[:batch].float().cpu().numpy()
        ok = bool(np.allclose(out, expected, atol=2e-2, rtol=1e-2))
        check = dict(ok=ok, max_abs_err=float(np.max(np.abs(out - expected))))
        print(f"[bench] oracle check ({best}): ok={ok} max_abs_err={check['max_abs_err']:.4g}",
              flush=True)
        if not ok:
            print("[bench] OUTPUT MISMATCH against the oracle", file=sys.stderr)
            sys.exit(3)

    # roofline: attention kernel alone, HIP events on its launch stream, rotating layers
    p = engine.plan
    stream = torch.cuda.current_stream(dev)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(args.kernel_launches)]
    engine.prepare()
    for i in range(args.kernel_launches):
        li = i % layers
        layer = engine.layers[li]
        x = fx[li]
        layer.counter.zero_()
        ev[i][0].record(stream)
        persistent_decode(p, layer, graph.q[li], x[1], x[2], graph.pages[li], graph.indptr[li],
                          c.head_dim ** -0.5, (x[1].stride(0), 0, x[1].stride(1), x[1].stride(2)),
                          (x[2].stride(0), 0, x[2].stride(1), x[2].stride(2)), (0, 0), True,
                          args.kernel)
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    durs = [a.elapsed_time(b) * 1000.0 for a, b in ev[len(ev) // 10:]]
    kern_us = statistics.mean(durs)
    achieved = bytes_per_layer / (kern_us * 1e-6) / 1e9
    kernel_name = engine.attention_kernel_name()
    roofline = dict(bound="hbm", achieved=round(achieved, 1), peak=PEAK_HBM_GBS, unit="GB/s",
                    frac=round(achieved / PEAK_HBM_GBS, 4),
                    traffic=measured_traffic(args.traffic_file, kernel_name, workers, bytes_per_layer),
                    attention_kernel=kernel_name,
                    kernel="persistent_decode", kernel_us=round(kern_us, 2),
                    algorithmic_bytes=bytes_per_layer)
    print(f"[bench] attention kernel alone ({best}): {kern_us:.2f} us  {achieved:.0f} GB/s", flush=True)

    if args.copy_calibration_mib:
        # a plain copy kernel of known size: N MiB read + N MiB written per launch
        n = args.copy_calibration_mib * (1 << 20) // 2
        a = torch.randn(n, device=dev).to(torch.bfloat16)
        b = torch.empty_like(a)
        for _ in range(5):
            torch.mul(a, 1, out=b)
        torch.cuda.synchronize()
        print(f"[bench] copy calibration: 5 x {args.copy_calibration_mib} MiB read+write", flush=True)

    cpu = None
    if not args.no_cpu_baseline:
        # the sample: the full layer (all requests) on host-resident fp32-upcast inputs
        for _ in range(2):
            t0 = time.perf_counter()
            OA.csr_attention(*host, lengths)
            cpu_times.append(time.perf_counter() - t0)
        t = statistics.median(cpu_times)
        cpu = dict(value=round(t * 1e6, 1), unit="us/layer", cores=1, kind="port",
                   sample=f"FP32 numpy oracle over the full layer ({batch} requests, "
                          f"{sum(lengths)} context tokens), median of 3, single thread",
                   tokens_per_s=round(batch / t, 2), kv_tokens_per_s=round(sum(lengths) / t, 1))
        print(f"[bench] cpu baseline: {t * 1e3:.1f} ms/layer", flush=True)

    r = results[best]
    line = {
        "metric": METRIC, "value": round(r["gbps"], 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(r["ms_per_step"], 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded lognormal contexts, N(0,1) bf16 q/K/V, permuted 1M-token pools)",
        "config": {"workload": "llama3-8b decode layer: B=64, 32q/8kv, D=128, bf16, CSR page 1, "
                               "lognormal(median 1024) contexts clipped [128,8192], 1M-token pool",
                   "batch": batch, "sum_context": sum(lengths), "layers_per_step": layers,
                   "schedule": best, "workers": workers, "kernel": args.kernel,
                   "splits_total": sum(splits)},
        "us_per_layer": round(r["us_per_layer"], 2),
        "pct_peak_hbm": round(100 * r["gbps"] / PEAK_HBM_GBS, 2),
        "tokens_per_s": round(batch / (r["us_per_layer"] * 1e-6), 1),
        "kv_tokens_per_s": round(sum(lengths) / (r["us_per_layer"] * 1e-6), 1),
        "schedules": {k: {kk: round(vv, 3) for kk, vv in v.items()} for k, v in results.items()},
        "check": check,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    text = json.dumps(line)
    if args.json_out:
        with open(args.json_out, "w") as f:
            f.write(text + "\n")
    print(text, flush=True)


if __name__ == "__main__":
    main()
