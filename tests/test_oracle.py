"""Pins the oracle before anything is checked against it.

* Plan stages (oracle/plan_spec.c) against the reference's own known-answer tests
  (tests/unit/test_planning.py:9-54 of the reference) and against the full
  sequences its CPU spec produced (tests/golden/plan_vectors.json).
* Device-only semantics (error flag, mode selection, R0 stop, uniform bypass)
  against closed forms from kernels/plan.py:16-20, 57-74.
* The FP32 attention oracle against closed forms (single token, equal keys, one
  dominant key) and against torch's scaled_dot_product_attention on the CPU.
* The merge oracle against the identity merge(split partials) == unsplit attention.
Several checks plant a mistake in the oracle's inputs to show the check can fail.
"""
import math
import types

import numpy as np
import pytest

from oracle import attention as OA
from oracle import plan as OP


def cfg(bcap=64, smax=16, max_context=32768, workers=108, hkv=8, block_kv=128):
    return types.SimpleNamespace(batch_capacity=bcap, max_splits=smax, max_context=max_context,
                                 workers=workers, kv_heads=hkv, block_kv=block_kv)


def split_hints(lengths, maximum=16):
    chunk = max(1, math.ceil(max(lengths, default=0) / maximum))
    return [max(1, min(maximum, math.ceil(n / chunk))) for n in lengths]


def oracle_records(lengths, splits, c):
    cs = OP.count_scan(lengths, splits, len(lengths), c.batch_capacity, c.max_splits,
                       c.max_context)
    rec = OP.emit_records(lengths, cs["counts"], cs["offsets"], cs["chunk"], c.batch_capacity,
                          c.max_splits, c.block_kv, c.batch_capacity * c.max_splits)
    n = cs["record_count"]
    rows = [[rec[k][i] for k in ("request", "split", "begin", "end", "weight")] for i in range(n)]
    return cs, rows


def buckets_of(c):
    return ((c.max_context + c.block_kv - 1) // c.block_kv - 1).bit_length() + 1


# --------------------------------------------------------------- reference KATs

@pytest.mark.parametrize("lengths,splits,records_count,pack_count", [
    ([512] * 24 + [8192] * 8, [1] * 24 + [16] * 8, 152, 1216),
    ([256] * 24 + [1536] * 4 + [16384] * 4, [1] * 24 + [2] * 4 + [16] * 4, 96, 705),
    (([256] * 24 + [1536] * 4 + [16384] * 4) * 2, ([1] * 24 + [2] * 4 + [16] * 4) * 2, 192, 1329),
])
def test_reference_task_geometry_kat(lengths, splits, records_count, pack_count):
    c = cfg()
    cs, rows = oracle_records(lengths, splits, c)
    assert cs["record_count"] == records_count == sum(cs["counts"]) == cs["offsets"][-1]
    op = OP.order_and_packs([r[4] for r in rows], len(rows), [], 4, c.kv_heads, c.workers,
                            buckets_of(c), c.batch_capacity * c.max_splits)
    assert op["num_packs"] == pack_count
    longest = max(r[4] for r in rows)
    covered = []
    for first, count in zip(op["pack_first"], op["pack_count"]):
        assert 1 <= count <= 4
        assert sum(rows[op["order"][t // c.kv_heads]][4] for t in range(first, first + count)) <= longest
        covered.extend(range(first, first + count))
    assert sorted(covered) == list(range(len(rows) * c.kv_heads))


def test_reference_tail_and_zero_lengths_kat():
    cs, rows = oracle_records([0, 1, 33, 513], [16, 16, 16, 2], cfg())
    assert cs["counts"][:4] == [0, 1, 2, 2]
    assert [(r[2], r[3]) for r in rows if r[0] == 3] == [(0, 288), (288, 513)]
    assert all(r[2] < r[3] for r in rows)


def test_reference_small_bucket_singletons_kat():
    c = cfg()
    _, rows = oracle_records([128, 1024], [1, 1], c)
    op = OP.order_and_packs([r[4] for r in rows], len(rows), [], 4, c.kv_heads, c.workers,
                            buckets_of(c), 1024)
    assert set(op["pack_count"]) == {1}


def test_reference_static_balance_kat():
    c = cfg(workers=4)
    _, rows = oracle_records([512] * 8, [1] * 8, c)
    heads, nxt = OP.greedy_static([r[4] for r in rows], len(rows), c.kv_heads, 4, 1024 * 8)
    lists = OP.walk_lists(heads, nxt)
    assert sorted(t for w in lists for t in w) == list(range(64))
    assert {len(w) for w in lists} == {16}


# --------------------------------------------------------------- golden full sequences

def test_oracle_matches_reference_sequences(plan_vectors):
    for case in plan_vectors:
        cc = case["config"]
        c = cfg(cc["batch_capacity"], cc["max_splits"], cc["max_context"], cc["workers"],
                cc["kv_heads"], cc["block_kv"])
        lengths, splits = case["lengths"], case["splits"]
        cs, rows = oracle_records(lengths, splits, c)
        assert cs["error"] == 0, case["name"]
        assert rows == case["records"], case["name"]
        assert cs["counts"][:len(lengths)] == case["counts"], case["name"]
        assert cs["offsets"][:len(lengths) + 1] == case["offsets"], case["name"]
        weights = [r[4] for r in rows]
        e = c.batch_capacity * c.max_splits
        for force, key in ((3, "packs_d1"), (4, "packs_d4")):
            op = OP.order_and_packs(weights, len(rows), [], force, c.kv_heads, c.workers,
                                    buckets_of(c), e)
            assert op["order"] == case["order"], case["name"]
            assert [list(p) for p in zip(op["pack_first"], op["pack_count"])] == case[key], case["name"]
        # device LPT (greedy_lists) and host heap LPT (greedy_static) give the reference lists
        heads, nxt = OP.greedy_lists(weights, len(rows), 2, c.kv_heads, c.workers, e * c.kv_heads)
        assert OP.walk_lists(heads, nxt) == case["static_lists"], case["name"]
        heads, nxt = OP.greedy_static(weights, len(rows), c.kv_heads, c.workers, e * c.kv_heads)
        assert OP.walk_lists(heads, nxt) == case["static_lists"], case["name"]


def test_golden_check_detects_planted_mistake(plan_vectors):
    case = next(c for c in plan_vectors if c["name"] == "B/w108")
    c = cfg()
    _, rows = oracle_records(case["lengths"], case["splits"], c)
    weights = [r[4] for r in rows]
    # plant: a smaller reserved singleton wave (workers - 8) changes the packs
    op = OP.order_and_packs(weights, len(rows), [], 4, c.kv_heads, c.workers - 8, buckets_of(c), 1024)
    assert [list(p) for p in zip(op["pack_first"], op["pack_count"])] != case["packs_d4"]
    # plant: a different split count changes the records
    _, rows2 = oracle_records(case["lengths"], [s + 1 if s < 16 else s for s in case["splits"]], c)
    assert rows2 != case["records"]


# --------------------------------------------------------------- device-only closed forms

def test_count_scan_error_and_inactive_rows():
    # active outside [0, bcap] -> error, no records, offsets all zero (plan.py:17, :20)
    for active in (-1, 5):
        cs = OP.count_scan([10, 20, 30, 40], [1, 1, 1, 1], active, 4, 16, 256)
        assert cs["error"] == 1 and cs["record_count"] == 0 and cs["offsets"] == [0] * 5
        assert cs["counts"] == [0] * 4
    # an invalid live row poisons the batch
    for bad in ([300, 1], [10, 0], [10, 17], [-1, 1]):
        cs = OP.count_scan([bad[0], 10], [bad[1], 1], 2, 4, 16, 256)
        assert cs["error"] == 1 and cs["record_count"] == 0
    # rows beyond active are not live: chunk 0, count 0, even if their data is invalid
    cs = OP.count_scan([64, 999999, 7, 7], [2, 0, 1, 1], 1, 4, 16, 256)
    assert cs["error"] == 0 and cs["counts"] == [2, 0, 0, 0] and cs["chunk"] == [32, 0, 0, 0]
    assert cs["offsets"] == [0, 2, 2, 2, 2]


def test_mode_selection_closed_forms():
    w, hkv, workers, buckets = [8, 1, 8, 1], 8, 108, 4
    rule_d4 = [[1, 10 ** 6, 101, 10000, 4]]
    assert OP.order_and_packs(w, 4, rule_d4, -1, hkv, workers, buckets, 16)["mode"] == 4
    # uniform bypass -> R1 even when a rule matches (plan.py:67-68)
    assert OP.order_and_packs([8, 8], 2, rule_d4, -1, hkv, workers, buckets, 16)["mode"] == 1
    # last matching rule wins (plan.py:61-66)
    two = rule_d4 + [[1, 10 ** 6, 100, 10000, 3]]
    assert OP.order_and_packs(w, 4, two, -1, hkv, workers, buckets, 16)["mode"] == 3
    # task bound excludes the rule -> default R1
    assert OP.order_and_packs(w, 4, [[1, 31, 101, 10000, 4]], -1, hkv, workers, buckets, 16)["mode"] == 1
    # force overrides the bypass (plan.py:69-70)
    op = OP.order_and_packs([8, 8], 2, [], 3, hkv, workers, buckets, 16)
    assert op["mode"] == 3 and op["num_packs"] == 16
    # R1 -> identity order, no packs
    op = OP.order_and_packs(w, 4, [], 1, hkv, workers, buckets, 16)
    assert op["order"] == [0, 1, 2, 3] and op["num_packs"] == 0
    # empty plan: default R1, no packs
    assert OP.order_and_packs([], 0, rule_d4, -1, hkv, workers, buckets, 16)["mode"] == 1


def test_forced_r0_stops_after_count_scan():
    c = cfg(bcap=4)
    plan = OP.full_plan([100, 0, 513, 7], [2, 1, 2, 1], 4, c, force=0)
    assert plan["mode"] == 0 and plan["num_packs"] == 0 and "request" not in plan
    assert plan["counts"] == [2, 0, 2, 1]


def test_greedy_lists_bruteforce_lpt():
    """Tiny inputs: every assignment step takes a (load, worker)-minimal worker and tasks are
    visited heaviest-first; brute force over the plan checks both facts."""
    rng = np.random.default_rng(7)
    for _ in range(20):
        n, hkv, workers = int(rng.integers(1, 7)), int(rng.integers(1, 4)), int(rng.integers(1, 6))
        weights = [int(x) for x in rng.integers(1, 5, size=n)]
        heads, nxt = OP.greedy_lists(weights, n, 2, hkv, workers, n * hkv)
        lists = OP.walk_lists(heads, nxt)
        owner = {t: w for w, ts in enumerate(lists) for t in ts}
        assert sorted(owner) == list(range(n * hkv))
        seq = sorted(range(n * hkv), key=lambda t: (-weights[t // hkv], t))
        loads = [0] * workers
        for t in seq:
            best = min(range(workers), key=lambda k: (loads[k], k))
            assert owner[t] == best
            loads[best] += weights[t // hkv]
        for ts in lists:
            assert ts == sorted(ts, key=lambda t: seq.index(t))


# --------------------------------------------------------------- attention oracle

def _rand(shape, rng):
    return rng.standard_normal(shape).astype(np.float32)


def test_attention_oracle_closed_forms():
    rng = np.random.default_rng(0)
    hq, hkv, d = 8, 2, 64
    q = _rand((1, hq, d), rng)
    k = _rand((5, 1, hkv, d), rng)
    v = _rand((5, 1, hkv, d), rng)
    pages = np.array([[3, 1, 4, 0, 2]])
    # single token -> its V row
    out = OA.paged_attention(q, k, v, pages, [1], 1)
    np.testing.assert_allclose(out[0], np.repeat(v[3, 0], hq // hkv, axis=0), rtol=1e-6)
    # identical keys -> mean of the gathered V rows
    k_same = np.repeat(k[:1], 5, axis=0)
    out = OA.paged_attention(q, k_same, v, pages, [4], 1)
    mean = v[[3, 1, 4, 0], 0].mean(axis=0)
    np.testing.assert_allclose(out[0], np.repeat(mean, hq // hkv, axis=0), rtol=1e-5, atol=1e-6)
    # one dominant key -> that V row
    k_dom = k.copy()
    k_dom[4, 0] = q[0, 0] * 50.0
    out = OA.paged_attention(q, k_dom, v, pages, [5], 1, scale=1.0)
    np.testing.assert_allclose(out[0, 0], v[4, 0, 0], rtol=1e-5, atol=1e-5)
    # L == 0 rows are zero
    assert not OA.paged_attention(q, k, v, pages, [0], 1).any()


def test_attention_oracle_matches_torch_sdpa():
    import torch
    rng = np.random.default_rng(1)
    b, hq, hkv, d, page = 3, 8, 2, 128, 4
    lengths = [13, 1, 30]
    q = _rand((b, hq, d), rng)
    k = _rand((20, page, hkv, d), rng)
    v = _rand((20, page, hkv, d), rng)
    pages = rng.permutation(20).reshape(2, 10).repeat(2, axis=0)[:b]
    out = OA.paged_attention(q, k, v, pages, lengths, page)
    for r, n in enumerate(lengths):
        tok = np.arange(n)
        key = torch.from_numpy(k[pages[r, tok // page], tok % page]).transpose(0, 1)  # [hkv, n, d]
        val = torch.from_numpy(v[pages[r, tok // page], tok % page]).transpose(0, 1)
        key = key.repeat_interleave(hq // hkv, 0)
        val = val.repeat_interleave(hq // hkv, 0)
        ref = torch.nn.functional.scaled_dot_product_attention(
            torch.from_numpy(q[r])[:, None], key, val)[:, 0]
        np.testing.assert_allclose(out[r], ref.numpy(), rtol=1e-4, atol=1e-5)
    # plant: a transposed head mapping (kv head h % hkv instead of h // group) must differ
    bad = k.copy()
    bad[..., 0, :], bad[..., 1, :] = k[..., 1, :], k[..., 0, :]
    assert not np.allclose(OA.paged_attention(q, bad, v, pages, lengths, page), out, atol=1e-3)


def test_csr_adapter_equals_paged():
    rng = np.random.default_rng(2)
    lengths = [5, 0, 9]
    q = _rand((3, 4, 64), rng)
    k = _rand((40, 2, 64), rng)
    v = _rand((40, 2, 64), rng)
    idx = rng.permutation(40)[:14]
    indptr = np.array([0, 5, 5, 14])
    out = OA.csr_attention(q, k, v, indptr, idx, lengths)
    pages = np.zeros((3, 9), dtype=np.int64)
    pages[0, :5], pages[2, :9] = idx[:5], idx[5:]
    np.testing.assert_allclose(out, OA.paged_attention(q, k[:, None], v[:, None], pages, lengths, 1),
                               rtol=1e-6)


def test_merge_of_split_partials_equals_unsplit_attention():
    rng = np.random.default_rng(3)
    c = cfg(bcap=3, smax=4, max_context=512, hkv=2)
    hq, d, page = 4, 64, 1
    lengths = [200, 33, 0]
    splits = [4, 2, 1]
    q = _rand((3, hq, d), rng)
    k = _rand((300, 1, 2, d), rng)
    v = _rand((300, 1, 2, d), rng)
    pages = np.zeros((3, 512), dtype=np.int64)
    perm = rng.permutation(300)
    pages[0, :200], pages[1, :33] = perm[:200], perm[200:233]
    cs, rows = oracle_records(lengths, splits, c)
    parts = OA.split_partials(q, k, v, pages, lengths, page, [r[:4] for r in rows], hq, c.max_splits)
    partial = np.full((3, hq, 4, d), np.nan, dtype=np.float32)
    lse = np.full((3, hq, 4), np.nan, dtype=np.float32)
    for (r, h, s), (p, l) in parts.items():
        partial[r, h, s], lse[r, h, s] = p, l
    merged = OP.merge_splits(partial, lse, cs["counts"], 0, 3, hq, d, 4)
    direct = OA.paged_attention(q, k, v, pages, lengths, page)
    np.testing.assert_allclose(merged, direct, rtol=1e-4, atol=1e-5)
    assert not merged[2].any()  # n == 0 row is exact zero despite NaN-poisoned slots
    assert np.isnan(OP.merge_splits(partial, lse, cs["counts"], 1, 3, hq, d, 4)).all()
    # plant: dropping the LSE weight (plain average of splits) must be caught
    flat = np.where(np.isnan(lse), lse, 0.0).astype(np.float32)
    assert not np.allclose(OP.merge_splits(partial, flat, cs["counts"], 0, 3, hq, d, 4)[0], direct[0],
                           atol=1e-3)


def test_threaded_oracle_matches_serial_oracle():
    """The CPU baseline's threaded restatement (every host core) computes what the serial
    oracle does: same gather, upcast and softmax, to float32 rounding."""
    import torch
    gen = torch.Generator().manual_seed(5)
    b, hq, hkv, d, page = 6, 8, 2, 128, 16
    lengths = [0, 1, 37, 130, 64, 5]
    pages = torch.randperm(60, generator=gen)[:b * 10].view(b, 10).to(torch.int32)
    q = torch.randn((b, hq, d), generator=gen).to(torch.bfloat16)
    k = torch.randn((60, page, hkv, d), generator=gen).to(torch.bfloat16)
    v = torch.randn((60, page, hkv, d), generator=gen).to(torch.bfloat16)
    serial = OA.paged_attention(q, k, v, pages, lengths, page)
    threaded = OA.paged_attention_threads(q, k, v, pages, lengths, page, threads=3)
    np.testing.assert_allclose(threaded, serial, rtol=1e-5, atol=1e-5)
    assert not threaded[0].any()
