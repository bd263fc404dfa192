"""hipGraph lifecycle: plan rebuilt on every replay, per-layer counters/scratch,
stable pointers, shrink/regrow, device mode switching, capacity errors."""
import os
import pytest
import torch

from oracle import attention as OA
from sglang_decode import workloads as W
from sglang_decode.config import DecodeConfig, Mode
from sglang_decode.planning.policy import PolicyRule
from sglang_decode.runtime.engine import DecodeEngine, PlanKey
from sglang_decode.runtime.graph import DecodeGraph

from gpu_util import close

pytestmark = pytest.mark.gpu


def test_graph_shrink_regrow_switch_modes_and_reset_layers():
    c = DecodeConfig(batch_capacity=32, max_context=1024)
    rules = [PolicyRule(1, c.task_capacity, 101, 10000, int(Mode.D4))]
    engine = DecodeEngine(c, layers=2, rules=rules)
    fixtures = [W.make_inputs(c, [1024] * 32, seed=40 + i) for i in range(2)]
    key = PlanKey("shared-sequence-order", "test-splits", (32, 8, 128))
    graph = DecodeGraph(engine, [key] * 2, [(x[1], x[2]) for x in fixtures])
    pointers = [(x.counter.data_ptr(), x.partial.data_ptr(), x.output.data_ptr()) for x in engine.layers]
    for step, batch in enumerate([32, 7, 1, 32]):
        lengths = [1024 if i % 3 == 0 else 33 for i in range(batch)]
        splits = [1] * batch
        graph.update([x[0][:batch] for x in fixtures], [x[3][:batch] for x in fixtures], lengths, splits)
        if step == 0:
            graph.capture()
        for layer in engine.layers:  # poison everything: every valid result must be rewritten
            layer.partial.fill_(float("nan"))
            layer.lse.fill_(float("nan"))
            layer.counter.fill_(100000)
        outputs = graph.replay()
        torch.cuda.synchronize()
        for layer, x in enumerate(fixtures):
            expected = OA.paged_attention(*x[:3], x[3], lengths, c.page_size)
            close(outputs[layer][:batch], expected[:batch])
        assert pointers == [(x.counter.data_ptr(), x.partial.data_ptr(), x.output.data_ptr())
                            for x in engine.layers]
        assert engine.plan.mode.item() == (Mode.R1 if batch == 1 else Mode.D4)


def test_capacity_and_layer_compatibility_before_capture():
    c = DecodeConfig(batch_capacity=2, max_context=1024)
    engine = DecodeEngine(c, layers=2)
    x = W.make_inputs(c, [17, 33])
    first = PlanKey("a", "s", (32, 8, 128))
    second = PlanKey("b", "s", (32, 8, 128))
    with pytest.raises(ValueError):
        DecodeGraph(engine, [first, second], [(x[1], x[2])] * 2)
    graph = DecodeGraph(engine, [first] * 2, [(x[1], x[2])] * 2)
    with pytest.raises(ValueError):
        graph.update([], [], [1, 1, 1], [1, 1, 1])
    with pytest.raises(ValueError):
        graph.update([x[0][:2]] * 2, [x[3][:2]] * 2, [17, 2000], [1, 1])


@pytest.mark.parametrize("mode", [Mode.R1, Mode.D1, Mode.STATIC])
def test_csr_graph_replay_shrinking_batches(mode):
    """Four layers over distinct pools; batch 64 -> 48 -> 17 -> 1 with contexts growing by one."""
    c = DecodeConfig(batch_capacity=64, max_splits=16, max_context=4096, page_size=1, workers=256)
    base = W.lognormal_lengths(64, 512, 32, 2048, seed=9)
    layers = 4
    pool = sum(base) + 64 * 8
    fx = [W.make_csr_inputs(c, [x + 3 for x in base], seed=70 + i, pool_tokens=pool)
          for i in range(layers)]
    engine = DecodeEngine(c, layers=layers, force_mode=mode)
    key = PlanKey("batch", "hints", (32, 8, 128))
    graph = DecodeGraph(engine, [key] * layers, [(x[1], x[2]) for x in fx],
                        index_capacity=[x[4].numel() for x in fx])
    for step, batch in enumerate([64, 48, 17, 1]):
        lengths = [x + step for x in base[:batch]]
        # each layer's kv_indices for this step: the first L tokens of each request's slots
        indptrs, indices = [], []
        for x in fx:
            full_ptr = x[3].cpu().tolist()
            idx = x[4].cpu()
            parts = [idx[full_ptr[r]:full_ptr[r] + lengths[r]] for r in range(batch)]
            ptr = torch.zeros(batch + 1, dtype=torch.int32)
            ptr[1:] = torch.cumsum(torch.tensor(lengths), 0)
            indptrs.append(ptr.cuda())
            indices.append(torch.cat(parts).cuda())
        graph.update([x[0][:batch] for x in fx], indices, lengths, W.split_hints(lengths, 16))
        if step == 0:
            graph.capture()
        for layer in engine.layers:
            layer.partial.fill_(float("nan"))
            layer.counter.fill_(7777)
        outs = graph.replay()
        torch.cuda.synchronize()
        for i, x in enumerate(fx):
            exp = OA.csr_attention(x[0], x[1], x[2], indptrs[i], indices[i], lengths)
            close(outs[i][:batch], exp[:batch])


def _csr_step(fx, lengths):
    """Per-layer kv_indptr / kv_indices of one step: the first L tokens of each request's
    slots in that layer's pool."""
    indptrs, indices = [], []
    for x in fx:
        full_ptr = x[3].cpu().tolist()
        idx = x[4]
        parts = [idx[full_ptr[r]:full_ptr[r] + lengths[r]] for r in range(len(lengths))]
        ptr = torch.zeros(len(lengths) + 1, dtype=torch.int32)
        ptr[1:] = torch.cumsum(torch.tensor(lengths), 0)
        indptrs.append(ptr.cuda())
        indices.append(torch.cat(parts))
    return indptrs, indices


def _oracle_layer_steps(x, steps, threads):
    """FP32 oracle of one layer at every step: the layer's fixture rows (each request's
    slots for its longest context) are copied to the host once, and each step's
    (lengths, batch) reads a prefix of every request's rows there, on `threads` host
    threads (oracle.attention.paged_attention_threads, pages of one token)."""
    full_ptr = x[3].cpu().tolist()
    rows = x[4].long()
    k, v = x[1][rows].cpu()[:, None], x[2][rows].cpu()[:, None]  # [tokens, 1, Hkv, D]
    q = x[0].cpu()
    outs = []
    for lengths in steps:
        pages = torch.zeros((len(lengths), max(lengths)), dtype=torch.int64)
        for r, n in enumerate(lengths):
            pages[r, :n] = torch.arange(full_ptr[r], full_ptr[r] + n)
        outs.append(OA.paged_attention_threads(q[:len(lengths)], k, v, pages, lengths, 1, threads=threads))
    return outs


def test_llama8b_32_layer_graph_shrinking_batches():
    """The 32-layer decode step under one hipGraph: 8B heads, batch 64 -> 48 -> 17 -> 1
    with contexts growing by one per step from a lognormal start (median 2048), the plan
    rebuilt on the device at every replay (a D4 rule for non-uniform batches; the uniform
    batch-1 step takes the device bypass to R1), per-layer counters and scratch; every
    layer of every step against the FP32 oracle; the host rejects an over-capacity step
    before touching the graph."""
    c = W.config_for("c5")
    base = W.c5_lengths()
    layers = 32
    rules = [PolicyRule(1, c.task_capacity, 101, 10000, int(Mode.D4))]
    steps = len(W.C5_BATCHES)
    pool = sum(base) + 64 * steps
    fx = [W.make_csr_inputs(c, [x + steps for x in base], seed=500 + i, pool_tokens=pool, device_pool=True)
          for i in range(layers)]
    engine = DecodeEngine(c, layers=layers, rules=rules)
    key = PlanKey("c5", "hints", (c.query_heads, c.kv_heads, c.head_dim))
    graph = DecodeGraph(engine, [key] * layers, [(x[1], x[2]) for x in fx],
                        index_capacity=[x[4].numel() for x in fx])
    results, steps_lengths = [], []
    for step, batch in enumerate(W.C5_BATCHES):
        lengths = [x + step for x in base[:batch]]
        indptrs, indices = _csr_step(fx, lengths)
        graph.update([x[0][:batch] for x in fx], indices, lengths, W.split_hints(lengths, c.max_splits))
        if step == 0:
            graph.capture()
        for layer in engine.layers:
            layer.partial.fill_(float("nan"))
        outs = graph.replay()
        torch.cuda.synchronize()
        assert engine.plan.mode.item() == (Mode.R1 if batch == 1 else Mode.D4)
        results.append([o[:batch].float().cpu() for o in outs])
        steps_lengths.append(lengths)
    threads = min(16, len(os.sched_getaffinity(0)))
    for i in range(layers):
        expected = _oracle_layer_steps(fx[i], steps_lengths, threads)
        for step, lengths in enumerate(steps_lengths):
            close(results[step][i], expected[step], msg=f"layer {i} step {step} batch {len(lengths)}")
        print(f"layer {i}: {len(steps_lengths)} steps within tolerance", flush=True)
    # over capacity: the host refuses before the graph is touched
    with pytest.raises(ValueError):
        graph.update([x[0][:1] for x in fx], [x[4][:1] for x in fx], [c.max_context + 1], [1])


@pytest.mark.parametrize("mode", [Mode.D4, Mode.R1])
def test_graph_replay_single_split_rows_from_the_attention(mode):
    """Batch capacity 128 x 32 query heads = 4096 merge rows, beyond one residency round
    of the merge (8 rows per CU on 256 CUs): each request's first split writes its rows and
    the merge only combines the multi-split ones.  Two layers under one hipGraph, batch
    128 -> 100 -> 3 with contexts growing by one and a mix of one and several splits per
    request; outputs, scratch and counters poisoned before every replay, so every row must
    be rewritten by the replay; every layer of every step against the FP32 oracle."""
    c = DecodeConfig(batch_capacity=128, max_splits=8, max_context=4096, page_size=1, workers=256)
    base = W.lognormal_lengths(128, 384, 16, 3000, seed=31)
    layers = 2
    fx = [W.make_csr_inputs(c, [x + 3 for x in base], seed=90 + i, pool_tokens=sum(base) + 128 * 4)
          for i in range(layers)]
    engine = DecodeEngine(c, layers=layers, force_mode=mode)
    if not engine.direct_first_split:
        pytest.skip("this device holds all 4096 merge rows in one residency round")
    key = PlanKey("batch", "hints", (32, 8, 128))
    graph = DecodeGraph(engine, [key] * layers, [(x[1], x[2]) for x in fx],
                        index_capacity=[x[4].numel() for x in fx])
    for step, batch in enumerate([128, 100, 3]):
        lengths = [x + step for x in base[:batch]]
        splits = W.split_hints(lengths, c.max_splits)
        assert 1 in splits and max(splits) > 1 or batch == 3
        print(f"graph direct mode={mode.name} step={step} batch={batch} "
              f"single={splits.count(1)}", flush=True)
        indptrs, indices = _csr_step(fx, lengths)
        graph.update([x[0][:batch] for x in fx], indices, lengths, splits)
        if step == 0:
            graph.capture()
        for layer in engine.layers:
            layer.partial.fill_(float("nan"))
            layer.output.fill_(float("nan"))
            layer.counter.fill_(7777)
        outs = graph.replay()
        torch.cuda.synchronize()
        for i, x in enumerate(fx):
            exp = OA.csr_attention(x[0], x[1], x[2], indptrs[i], indices[i].cuda(), lengths)
            close(outs[i][:batch], exp[:batch], msg=f"layer {i} step {step}")
            assert not outs[i][batch:].float().abs().sum().item()  # rows past the batch: zeros


def test_graph_many_replays_random_steps():
    """One captured two-layer step replayed 60 times, each step a fresh random batch (1-32
    requests, contexts 1-2048, 1-8 splits each, D1 forced): no state leaks from one replay
    into the next -- claim counters back at zero after every replay, and every sixth step's
    outputs against the FP32 oracle."""
    c = DecodeConfig(batch_capacity=32, max_splits=8, max_context=2048, page_size=1, workers=512)
    layers = 2
    full = [2048] * 32
    fx = [W.make_csr_inputs(c, full, seed=600 + i, pool_tokens=32 * 2048) for i in range(layers)]
    engine = DecodeEngine(c, layers=layers, force_mode=Mode.D1)
    key = PlanKey("batch", "hints", (32, 8, 128))
    graph = DecodeGraph(engine, [key] * layers, [(x[1], x[2]) for x in fx],
                        index_capacity=[x[4].numel() for x in fx])
    rng = torch.Generator().manual_seed(77)
    for step in range(60):
        batch = int(torch.randint(1, 33, (1,), generator=rng))
        lengths = torch.randint(1, 2049, (batch,), generator=rng).tolist()
        splits = torch.randint(1, 9, (batch,), generator=rng).tolist()
        indptrs, indices = _csr_step(fx, lengths)
        graph.update([x[0][:batch] for x in fx], indices, lengths, splits)
        if step == 0:
            graph.capture()
        outs = graph.replay()
        torch.cuda.synchronize()
        assert not engine.sync.any().item(), step
        if step % 6 == 0:
            print(f"replay {step}: batch {batch}", flush=True)
            for i, x in enumerate(fx):
                exp = OA.csr_attention(x[0], x[1], x[2], indptrs[i], indices[i].cuda(), lengths)
                close(outs[i][:batch], exp[:batch], msg=f"replay {step} layer {i}")
