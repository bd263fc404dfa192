"""The reference's GPU tests (tests/gpu/test_decode.py:12-56, tests/gpu/test_graph.py:13-51),
restated against this package through the reference's own import paths -- the oracle as
sglang_decode.reference.attention and the harness as benchmarks.workloads (test-side
aliases, tests/conftest.py) -- to show a caller of the reference switches without edits.
Tolerance: 2e-2 abs / 1e-2 rel against the FP32 oracle (tighter in rtol than the
reference's 2e-2)."""
import pytest
import torch

from benchmarks.workloads import WORKLOADS, make_inputs, split_hints, update_plan
from sglang_decode.config import DecodeConfig, Mode
from sglang_decode.planning.policy import PolicyRule
from sglang_decode.planning.reference import bucket_order, make_packs, split_records
from sglang_decode.reference.attention import paged_attention
from sglang_decode.runtime.engine import DecodeEngine, PlanKey
from sglang_decode.runtime.graph import DecodeGraph

pytestmark = pytest.mark.gpu


def _close(actual, expected):
    torch.testing.assert_close(actual.float().cpu(), expected, atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("mode", list(Mode))
@pytest.mark.parametrize("lengths", [[0, 1, 17, 33, 257, 513], WORKLOADS["B"]])
def test_outputs_records_order_and_packs(mode, lengths):
    c = DecodeConfig()
    engine = DecodeEngine(c, force_mode=mode)
    inputs = make_inputs(c, lengths)
    update_plan(engine, lengths)
    engine.layers[0].partial.fill_(float("nan"))
    engine.layers[0].lse.fill_(float("nan"))
    engine.prepare()
    out = engine.execute(*inputs)
    n = len(lengths)
    _close(out[:n], paged_attention(*inputs[:3], inputs[3], lengths, c.page_size)[:n])
    records, counts, _ = split_records(lengths, split_hints(lengths), c)
    p = engine.plan
    assert p.error.item() == 0 and p.record_count.item() == len(records)
    assert p.counts[:n].tolist() == counts
    if mode != Mode.R0:
        assert p.request[:len(records)].tolist() == [r.request for r in records]
        assert p.begin[:len(records)].tolist() == [r.begin for r in records]
    if mode in (Mode.D1, Mode.D4):
        order = bucket_order(records)
        packs = make_packs(records, order, c.kv_heads, c.workers, pack_limit=1 if mode == Mode.D1 else 4)
        assert p.order[:len(records)].tolist() == order
        k = p.num_packs.item()
        assert list(zip(p.pack_first[:k].tolist(), p.pack_count[:k].tolist())) == packs


def test_graph_shrink_regrow_and_switch_modes():
    c = DecodeConfig(batch_capacity=32, max_context=1024)
    rules = [PolicyRule(1, c.task_capacity, 101, 10000, int(Mode.D4))]
    engine = DecodeEngine(c, layers=2, rules=rules)
    fixtures = [make_inputs(c, [1024] * 32, seed=40 + i) for i in range(2)]
    graph = DecodeGraph(engine, [PlanKey("seq", "splits", (32, 8, 128))] * 2, [(x[1], x[2]) for x in fixtures])
    held = [(x.counter.data_ptr(), x.partial.data_ptr(), x.output.data_ptr()) for x in engine.layers]
    for step, batch in enumerate([32, 7, 1, 20]):
        # one split per request and two lengths: non-uniform work (D4 through the rule)
        # except for the single request, which the device plan sends to R1
        lengths = [33 if i % 3 else 1024 for i in range(batch)]
        graph.update([x[0][:batch] for x in fixtures], [x[3][:batch] for x in fixtures], lengths, [1] * batch)
        if step == 0:
            graph.capture()
        for layer in engine.layers:  # every valid result must be rewritten by the replay
            layer.partial.fill_(float("nan"))
            layer.lse.fill_(float("nan"))
            layer.counter.fill_(100000)
        outs = graph.replay()
        torch.cuda.synchronize()
        for layer, x in enumerate(fixtures):
            _close(outs[layer][:batch], paged_attention(x[0], x[1], x[2], x[3], lengths, c.page_size)[:batch])
        assert held == [(x.counter.data_ptr(), x.partial.data_ptr(), x.output.data_ptr()) for x in engine.layers]
        assert engine.plan.mode.item() == (Mode.R1 if batch == 1 else Mode.D4)
