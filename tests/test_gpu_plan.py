"""Device plan parity: every stage of the GPU plan is bit-exact against the oracle
(which tests/test_oracle.py pins to the reference's own planning results)."""
import pytest
import torch

from oracle import plan as OP
from sglang_decode import workloads as W
from sglang_decode.config import DecodeConfig, Mode
from sglang_decode.planning.builder import build_plan
from sglang_decode.planning.policy import PolicyRule
from sglang_decode.runtime.workspace import PlanBuffers

from gpu_util import assert_plan_equal, cfg_ns, read_plan

pytestmark = pytest.mark.gpu

FORCES = [-1, 0, 1, 2, 3, 4]


def load(plan, lengths, splits, active=None):
    c = plan.config
    n = len(lengths)
    lw = torch.zeros(c.batch_capacity, dtype=torch.int32)
    sw = torch.ones(c.batch_capacity, dtype=torch.int32)
    lw[:n] = torch.tensor(lengths, dtype=torch.int32)
    sw[:n] = torch.tensor(splits, dtype=torch.int32)
    plan.lengths.copy_(lw)
    plan.splits.copy_(sw)
    plan.active.fill_(n if active is None else active)


def poison(plan):
    for name in ("counts", "offsets", "chunk", "request", "split", "begin", "end", "weight", "order",
                 "pack_first", "pack_count", "static_head", "static_next", "record_count",
                 "num_packs", "mode", "error"):
        getattr(plan, name).fill_(-7)


def run_case(c, lengths, splits, force, fused, rules=(), active=None, name=""):
    plan = PlanBuffers(c, "cuda", rules)
    load(plan, lengths, splits, active)
    poison(plan)
    build_plan(plan, force, fused=fused)
    dev = read_plan(plan)
    act = len(lengths) if active is None else active
    lw = list(lengths) + [0] * (c.batch_capacity - len(lengths))
    sw = list(splits) + [1] * (c.batch_capacity - len(splits))
    flat_rules = [[r.min_tasks, r.max_tasks, r.min_ratio, r.max_ratio, r.mode] for r in rules]
    ref = OP.full_plan(lw, sw, act, cfg_ns(c), flat_rules, force)
    if force == 0:
        ref = dict(ref)  # records are not emitted under forced R0
    assert_plan_equal(dev, ref, c, act, f"{name} force={force} fused={fused}")
    return dev


@pytest.mark.parametrize("fused", [True, False])
def test_plan_matches_oracle_on_benchmark_configs(fused):
    for name in ("c1", "c2", "c3", "c4", "c5"):
        c = W.config_for(name)
        lengths = W.lengths_for(name)
        splits = W.splits_for(name, lengths, c)
        for force in FORCES:
            run_case(c, lengths, splits, force, fused, name=name)


@pytest.mark.parametrize("fused", [True, False])
def test_plan_matches_reference_golden_cases(plan_vectors, fused):
    for case in plan_vectors:
        cc = case["config"]
        c = DecodeConfig(batch_capacity=cc["batch_capacity"], max_splits=cc["max_splits"],
                         max_context=cc["max_context"], workers=cc["workers"],
                         kv_heads=cc["kv_heads"], query_heads=cc["kv_heads"] * 4)
        for force in (3, 4):
            dev = run_case(c, case["lengths"], case["splits"], force, fused, name=case["name"])
            n = len(case["records"])
            assert [[dev[k][i] for k in ("request", "split", "begin", "end", "weight")]
                    for i in range(n)] == case["records"]
            assert dev["order"][:n] == case["order"]
            packs = case["packs_d4" if force == 4 else "packs_d1"]
            assert [list(p) for p in zip(dev["pack_first"][:dev["num_packs"]],
                                         dev["pack_count"][:dev["num_packs"]])] == packs
        dev = run_case(c, case["lengths"], case["splits"], 2, fused, name=case["name"])
        assert OP.walk_lists(dev["static_head"], dev["static_next"]) == case["static_lists"]


@pytest.mark.parametrize("fused", [True, False])
def test_plan_error_paths(fused):
    c = DecodeConfig(batch_capacity=8, max_context=1024, workers=16)
    for lengths, splits, active in (([10, 2000], [1, 1], None), ([10, 20], [1, 17], None),
                                    ([10, 20], [0, 1], None), ([-3, 5], [1, 1], None),
                                    ([10, 20], [1, 1], 9), ([10, 20], [1, 1], -1)):
        dev = run_case(c, lengths, splits, -1, fused, active=active)
        assert dev["error"] == 1 and dev["record_count"] == 0


@pytest.mark.parametrize("fused", [True, False])
def test_plan_rules_and_bypass(fused):
    c = DecodeConfig(batch_capacity=32, max_context=1024, workers=108)
    rules = [PolicyRule(1, c.task_capacity, 101, 10000, int(Mode.D4))]
    for batch in (32, 7, 1):
        lengths = [1024 if i % 3 == 0 else 33 for i in range(batch)]
        dev = run_case(c, lengths, [1] * batch, -1, fused, rules=rules)
        assert dev["mode"] == (Mode.R1 if batch == 1 else Mode.D4)
    static_rule = [PolicyRule(0, 10 ** 6, 100, 10000, int(Mode.STATIC))]
    dev = run_case(c, [1024, 33, 33], [1, 1, 1], -1, fused, rules=static_rule)
    assert dev["mode"] == Mode.STATIC


def test_plan_zero_batch_and_edges():
    c = DecodeConfig(batch_capacity=64, max_context=32768, workers=256)
    for lengths in ([], [0], [0, 0, 0], [1], [32768], [31, 32, 33, 63, 64, 65]):
        splits = W.split_hints(lengths, 16) if lengths else []
        for force in FORCES:
            run_case(c, lengths, splits, force, True)


def run_csr_case(c, lengths, splits, force, name=""):
    """sgd_build_plan_csr: the plan built from (kv_indptr, num_kv_splits, batch) inside the
    launch equals the oracle's plan of those rows, and the plan's lengths / splits rows <
    batch and active hold what the reference adapter's copies would (integrations/
    sglang_backend.py:98-99); rows >= batch are not touched."""
    plan = PlanBuffers(c, "cuda")
    for t in (plan.lengths, plan.splits, plan.active):
        t.fill_(-5)
    poison(plan)
    n = len(lengths)
    indptr = torch.zeros(n + 4, dtype=torch.int32)  # entries past batch + 1 must not matter
    indptr[1:n + 1] = torch.cumsum(torch.tensor(lengths, dtype=torch.int64), 0).to(torch.int32)
    indptr[n + 1:] = -999
    sp = torch.tensor(list(splits) + [77] * 3, dtype=torch.int32)
    build_plan(plan, force, csr_metadata=(indptr.cuda(), sp.cuda(), n))
    dev = read_plan(plan)
    lw = list(lengths) + [0] * (c.batch_capacity - n)
    sw = list(splits) + [1] * (c.batch_capacity - n)
    assert_plan_equal(dev, OP.full_plan(lw, sw, n, cfg_ns(c), [], force), c, n, f"{name} force={force} csr")
    assert plan.lengths[:n].tolist() == list(lengths) and plan.splits[:n].tolist() == list(splits)
    assert (plan.lengths[n:] == -5).all() and (plan.splits[n:] == -5).all() and plan.active.item() == n
    return dev


def test_plan_from_csr_metadata_matches_oracle():
    for name in ("c1", "c2", "c3", "c5"):
        c = W.config_for(name)
        lengths = W.lengths_for(name)
        splits = W.splits_for(name, lengths, c)
        for force in FORCES:
            run_csr_case(c, lengths, splits, force, name)
            run_csr_case(c, lengths[:len(lengths) // 2 + 1], splits[:len(lengths) // 2 + 1], force, name)
    c = DecodeConfig(batch_capacity=8, max_context=1024, workers=16)
    for force in FORCES:
        run_csr_case(c, [], [], force, "empty")
    # invalid rows: a decreasing kv_indptr (negative length), split counts outside [1, 16]
    for lengths, splits in (([10, -3, 5], [1, 1, 1]), ([10, 20], [1, 17]), ([10, 20], [0, 1])):
        dev = run_csr_case(c, lengths, splits, -1, "invalid")
        assert dev["error"] == 1 and dev["record_count"] == 0


def test_plan_from_csr_metadata_under_graph_replay():
    """The adapter's use under graph capture: one captured build reading fixed kv_indptr /
    num_kv_splits buffers whose contents change between replays (eager copies in between);
    every replay's plan equals the oracle plan of the current contents."""
    c = DecodeConfig(batch_capacity=8, max_context=1024, workers=16)
    plan = PlanBuffers(c, "cuda")
    sync = torch.zeros(2, dtype=torch.int32, device="cuda")
    batch = 5
    indptr = torch.zeros(batch + 1, dtype=torch.int32, device="cuda")
    splits = torch.ones(batch, dtype=torch.int32, device="cuda")

    def fill(lengths, sp):
        ip = torch.zeros(batch + 1, dtype=torch.int32)
        ip[1:] = torch.cumsum(torch.tensor(lengths), 0)
        indptr.copy_(ip)
        splits.copy_(torch.tensor(sp, dtype=torch.int32))

    steps = [([100, 1024, 3, 0, 512], [2, 16, 1, 1, 4]), ([1, 1, 1, 1, 1], [1, 1, 1, 1, 1]),
             ([900, 17, 640, 33, 1000], [8, 1, 5, 2, 16]), ([1024] * 5, [16] * 5)]
    fill(*steps[0])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        build_plan(plan, -1, counters=sync, csr_metadata=(indptr, splits, batch))
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            build_plan(plan, -1, counters=sync, csr_metadata=(indptr, splits, batch))
    torch.cuda.synchronize()
    for lengths, sp in steps + steps[:1]:
        fill(lengths, sp)
        poison(plan)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        lw, sw = lengths + [0] * (c.batch_capacity - batch), sp + [1] * (c.batch_capacity - batch)
        assert_plan_equal(read_plan(plan), OP.full_plan(lw, sw, batch, cfg_ns(c)), c, batch, str(lengths))
        assert plan.lengths[:batch].tolist() == lengths and plan.active.item() == batch


def test_plan_from_csr_metadata_rejects_bad_arguments():
    c = DecodeConfig(batch_capacity=8, max_context=1024, workers=16)
    plan = PlanBuffers(c, "cuda")
    indptr = torch.zeros(9, dtype=torch.int32, device="cuda")
    splits = torch.ones(8, dtype=torch.int32, device="cuda")
    for meta in ((indptr, splits, 9), (indptr, splits, -1), (indptr[:3], splits, 3), (indptr.long(), splits, 2),
                 (indptr, splits.cpu(), 2)):
        with pytest.raises(ValueError):
            build_plan(plan, -1, csr_metadata=meta)


def test_fused_plan_clears_counters():
    c = W.config_for("c1")
    plan = PlanBuffers(c, "cuda")
    load(plan, [17, 200], [1, 2])
    counters = torch.full((5,), 1234, dtype=torch.int32, device="cuda")
    build_plan(plan, -1, counters=counters)
    assert counters.tolist() == [0] * 5


def expected_table(ref, c, mode):
    """The dispatch table from the oracle plan: R1/STATIC task t (record t / Hkv; R1's
    order is the identity), D1/D4 pack u (its first task's record through the order)."""
    hkv = c.kv_heads
    total = ref["record_count"] * hkv
    fields = lambda rec: [ref[k][rec] for k in ("request", "split", "begin", "end")]
    if mode in (1, 2):
        if mode == 1:
            assert ref["order"][:ref["record_count"]] == list(range(ref["record_count"]))
        return [[t, 1] + fields(t // hkv) + [t % hkv, 1] for t in range(total)]
    if mode in (3, 4):
        rows = []
        for u in range(ref["num_packs"]):
            first, count = ref["pack_first"][u], ref["pack_count"][u]
            rows.append([first, count] + fields(ref["order"][first // hkv]) + [first % hkv, 2])
        return rows
    return []


@pytest.mark.parametrize("force", [0, 1, 2, 3, 4])
def test_dispatch_table_matches_oracle(force):
    """sgd_build_plan's dispatch table: one entry per unit, resolved exactly as the
    attention dispatch resolves it (pack -> order -> record); nothing past the units."""
    for name in ("c1", "c2", "c3", "c5"):
        for workers in (7, 256):
            c = W.config_for(name, workers=workers)
            lengths = W.lengths_for(name)
            splits = W.split_hints(lengths, c.max_splits)
            plan = PlanBuffers(c, "cuda")
            load(plan, lengths, splits)
            plan.dispatch.fill_(-9)
            build_plan(plan, force)
            assert plan.dispatch_valid
            lw = list(lengths) + [0] * (c.batch_capacity - len(lengths))
            sw = list(splits) + [1] * (c.batch_capacity - len(splits))
            ref = OP.full_plan(lw, sw, len(lengths), cfg_ns(c), [], force)
            exp = expected_table(ref, c, force)
            got = plan.dispatch.cpu()
            assert got[:len(exp)].tolist() == exp, (name, workers)
            assert (got[len(exp):] == -9).all(), (name, workers)
    build_plan(plan, force, fused=False)
    assert not plan.dispatch_valid  # the stage launches write no dispatch table
