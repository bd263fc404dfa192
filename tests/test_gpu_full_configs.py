"""Parity at the benchmark configurations' full sizes, every request, on the product's
defaults (AUTO kernel, two workers per CU), against the FP32 oracle (2e-2 abs / 1e-2 rel):

* Llama-3-8B heads, batch 64, CSR page 1, lognormal lengths (median 1024): every schedule;
* the skewed batch: 128 requests, 2 x 32768 + 126 x U[32, 512], up to 64 splits of at
  most 512 tokens: D1 and D4;
* Llama-3-70B heads, batch 32, page 16, lengths U[2048, 16384]: every schedule in bf16,
  D1 and D4 in fp16.

Partials and LSEs are NaN-poisoned before each launch, the plan's error flag, record
count and per-row counts are compared with the planning spec, and the per-layer claim
counters must be back at zero afterwards (reference: tests/gpu/test_decode.py:12-39)."""
import os

import pytest
import torch

from oracle import attention as OA
from sglang_decode import workloads as W
from sglang_decode.config import Mode, default_workers
from sglang_decode.planning.reference import split_records
from sglang_decode.runtime.engine import DecodeEngine

from gpu_util import close

pytestmark = pytest.mark.gpu

_CACHE = {}


def workload(name, dtype=torch.bfloat16):
    key = (name, dtype)
    if key not in _CACHE:
        _CACHE.clear()  # one configuration's pools on the device at a time
        torch.cuda.empty_cache()
        c = W.config_for(name, workers=default_workers())
        lengths = W.lengths_for(name)
        splits = W.splits_for(name, lengths, c)
        if c.page_size == 1:
            q, k, v, indptr, indices = W.make_csr_inputs(c, lengths, seed=61, dtype=dtype)
            expected = OA.csr_attention(q, k, v, indptr, indices, lengths)
            inputs = (q, k, v, indices)
        else:
            q, k, v, pages = W.make_inputs(c, lengths, seed=61, dtype=dtype)
            threads = min(16, len(os.sched_getaffinity(0)))
            expected = OA.paged_attention_threads(q.cpu(), k.cpu(), v.cpu(), pages.cpu(), lengths, c.page_size,
                                                  threads=threads)
            inputs, indptr = (q, k, v, pages), None
        _CACHE[key] = (c, lengths, splits, inputs, indptr, expected)
    return _CACHE[key]


def check(name, mode, dtype=torch.bfloat16):
    c, lengths, splits, inputs, indptr, expected = workload(name, dtype)
    print(f"{name} mode={Mode(mode).name} dtype={dtype} batch={len(lengths)} total={sum(lengths)}", flush=True)
    engine = DecodeEngine(c, dtype=dtype, force_mode=mode)
    W.update_plan(engine, lengths, splits)
    engine.layers[0].partial.fill_(float("nan"))
    engine.layers[0].lse.fill_(float("nan"))
    engine.prepare()
    out = engine.execute(*inputs, indptr=indptr)
    torch.cuda.synchronize()
    records, counts, _ = split_records(lengths, splits, c)
    assert engine.plan.error.item() == 0
    assert engine.plan.record_count.item() == len(records)
    assert engine.plan.counts[:len(lengths)].tolist() == counts
    assert engine.sync.abs().sum().item() == 0  # claim / finished counters back at zero
    close(out[:len(lengths)], expected[:len(lengths)], msg=f"{name} {Mode(mode).name} {dtype}")
    return engine


@pytest.mark.parametrize("mode", list(Mode))
def test_llama8b_batch64_every_request(mode):
    check("c2", mode)


@pytest.mark.parametrize("mode", [Mode.D1, Mode.D4])
def test_skewed_batch128_every_request(mode):
    engine = check("c3", mode)
    assert max(engine.plan.counts.tolist()) == 64  # the two long requests use all 64 splits


# every schedule in bf16, the claiming ones in fp16 too (grouped by dtype: one oracle each)
C4_CASES = [(torch.bfloat16, m) for m in Mode] + [(torch.float16, Mode.D1), (torch.float16, Mode.D4)]


@pytest.mark.parametrize("dtype,mode", C4_CASES, ids=[f"{str(d)[6:]}-{m.name}" for d, m in C4_CASES])
def test_llama70b_paged_batch32_every_request(dtype, mode):
    engine = check("c4", mode, dtype)
    assert engine.attention_kernel_name() == "mfma"


def test_llama8b_batch64_host_static_every_request():
    """STATIC_HOST at the reference benchmark's boundary (benchmarks/bench_decode.py:14-30):
    the host LPT lists uploaded from pinned memory over the R1 plan, on every request of
    the batch-64 layer, twice in a row (the second call re-plans into the same staging
    buffers).  The installed lists equal the planning spec's, the mode is STATIC, and the
    output is within tolerance of the FP32 oracle."""
    from sglang_decode.planning.host_static import HostStatic
    from sglang_decode.planning.reference import greedy_static, lists_to_links
    c, lengths, splits, inputs, indptr, expected = workload("c2")
    engine = DecodeEngine(c, force_mode=Mode.R1)
    W.update_plan(engine, lengths, splits)
    hs = HostStatic(engine)
    records, _, _ = split_records(lengths, splits, c)
    heads, links = lists_to_links(greedy_static(records, c.kv_heads, c.workers), c.workers, c.task_capacity)
    for _ in range(2):
        engine.layers[0].partial.fill_(float("nan"))
        hs.prepare(lengths, splits)
        out = engine.execute(*inputs, indptr=indptr)
        torch.cuda.synchronize()
        assert engine.plan.mode.item() == int(Mode.STATIC)
        assert engine.plan.static_head.tolist() == heads
        assert engine.plan.static_next.tolist() == links
        close(out[:len(lengths)], expected[:len(lengths)], msg="c2 STATIC_HOST")


@pytest.mark.parametrize("name,kernel", [("c2", "auto"), ("c3", "auto"), ("c4", "auto"), ("c2", "generic")])
def test_single_split_rows_from_the_attention_equal_the_merge(name, kernel):
    """With direct first-split writes (the engine's choice when the merge rows outnumber one
    residency round, C3 here; forced on for the others) each request's first split also
    writes its rows and the merge takes only the multi-split ones (sgd_merge_splits_min,
    min_splits 2).  Bit for bit the same output as the reference's order -- every split to
    its slot, every row merged (sgd_merge_splits) -- on each kernel; the split slots are
    still all written."""
    from sglang_decode.kernels.attention import checked_layout, persistent_decode
    from sglang_decode.kernels.merge import merge_splits
    c, lengths, splits, inputs, indptr, expected = workload(name)
    engine = DecodeEngine(c, force_mode=Mode.D1, kernel=kernel)
    assert engine.direct_first_split == (name == "c3")  # 4096 merge rows > 8 per CU x 256 CUs
    engine.direct_first_split = True
    W.update_plan(engine, lengths, splits)
    engine.prepare()
    layer = engine.layers[0]
    layer.output.fill_(float("nan"))
    layer.partial.fill_(float("nan"))
    direct = engine.execute(*inputs, indptr=indptr).clone()
    slots = layer.partial.clone()
    records, counts, _ = split_records(lengths, splits, c)
    assert name == "c4" or sum(1 for n in counts if n == 1) > 0  # c4: every request has several splits
    layer.output.fill_(float("nan"))
    layer.partial.fill_(float("nan"))
    ks, vs, pts, csr = checked_layout(c, *inputs, indptr, layer.output.dtype)
    persistent_decode(engine.plan, layer, *inputs, indptr, c.head_dim ** -0.5, ks, vs, pts, csr, kernel,
                      write_single=False)
    merge_splits(engine.plan, layer, min_splits=1)
    torch.cuda.synchronize()
    n = len(lengths)
    assert torch.equal(direct[:n].view(torch.int16), layer.output[:n].view(torch.int16)), name
    assert torch.equal(slots.view(torch.int32), layer.partial.view(torch.int32))
    close(direct[:n], expected[:n], msg=f"{name} {kernel}")
