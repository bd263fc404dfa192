"""The CSR metadata producer (csrc/csr_metadata.hip, sglang_decode/kernels/csr_metadata.py).

CPU: the oracle pinned by what fixes it -- kv_indptr by its closed form (prefix sums,
last entry = sum of the lengths), kv_indices by brute force over the table, split counts
against the reference harness fixture rule as the package restates it
(sglang_decode.workloads.split_hints, which the plan's golden sequences use) and its
documented boundaries, and the invalid-row and capacity rules.
GPU: the launch bit-exact against the oracle (int32/int64 inputs, empty and invalid rows,
an empty batch, a total beyond the capacity, the largest batch), its plan outputs feeding
sgd_build_plan, and attention over the produced metadata against the FP32 oracle."""
import numpy as np
import pytest
import torch

from oracle import csr_metadata as OM
from sglang_decode import workloads as W


def table(rows, cols, seed):
    r = np.random.Generator(np.random.PCG64(seed))
    return r.permutation(rows * cols).reshape(rows, cols).astype(np.int32)


def test_oracle_closed_forms_and_brute_force():
    t = table(9, 50, 1)
    lens, pool = [5, 0, 50, 17, 1], [3, 8, 0, 3, 7]
    m = OM.csr_metadata(lens, pool, t, 16, 10 ** 6)
    assert m["kv_indptr"] == [0, 5, 5, 55, 72, 73] and m["error"] == 0
    assert len(m["kv_indices"]) == m["kv_indptr"][-1] == sum(lens)
    for i, (L, p) in enumerate(zip(lens, pool)):  # slot j of row i is table[pool_i, j]
        for j in range(L):
            assert m["kv_indices"][m["kv_indptr"][i] + j] == t[p, j]
    assert m["num_kv_splits"] == W.split_hints(lens, 16)


def test_oracle_split_rule_boundaries():
    # chunk = ceil(maxL / S): a row one token past a chunk multiple takes one more split
    assert OM.harness_splits([1024, 64, 65, 1], 16) == [16, 1, 2, 1]
    assert OM.harness_splits([0, 0], 8) == [1, 1] and OM.harness_splits([], 8) == []
    assert OM.harness_splits([7, 3], 16) == [7, 3]  # chunk 1: one split per token up to S


def test_oracle_invalid_rows_and_capacity():
    t = table(4, 10, 2)
    m = OM.csr_metadata([3, -1, 11, 2, 4], [0, 1, 2, 9, 3], t, 4, 100)
    assert m["lengths"] == [3, 0, 0, 0, 4] and m["error"] == 1 and m["kv_indptr"][-1] == 7
    m = OM.csr_metadata([3, 4], [0, 1], t, 4, 6)  # 7 > capacity 6
    assert m["lengths"] == [0, 0] and m["kv_indptr"] == [0, 0, 0] and m["error"] == 1
    assert m["num_kv_splits"] == [1, 1]


def test_entry_point_declared_and_exported():
    from sglang_decode import _lib
    assert hasattr(_lib.lib(), "sgd_csr_metadata")


# ------------------------------------------------------------------ GPU

def run(lens, pool, t, smax, capacity, dtype=torch.int32, plan=None):
    from sglang_decode.kernels.csr_metadata import csr_metadata
    dev = "cuda"
    b = len(lens)
    indptr = torch.full((b + 3,), -9, dtype=torch.int32, device=dev)
    indices = torch.full((capacity,), -9, dtype=torch.int32, device=dev)
    splits = torch.full((b + 2,), -9, dtype=torch.int32, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    csr_metadata(torch.tensor(lens, dtype=dtype, device=dev), torch.tensor(pool, dtype=dtype, device=dev),
                 torch.from_numpy(t).to(dev), smax, indptr, indices, splits, plan=plan, error=err)
    torch.cuda.synchronize()
    ref = OM.csr_metadata(lens, pool, t, smax, capacity)
    n = ref["kv_indptr"][-1]
    assert indptr[:b + 1].tolist() == ref["kv_indptr"] and indptr[b + 1:].tolist() == [-9, -9]
    assert indices[:n].tolist() == ref["kv_indices"] and (indices[n:] == -9).all()
    assert splits[:b].tolist() == ref["num_kv_splits"] and err.item() == ref["error"]
    return ref


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_metadata_matches_oracle(dtype):
    t = table(300, 4096, 3)
    r = np.random.Generator(np.random.PCG64(4))
    for b in (1, 7, 64, 257):
        lens = [int(x) for x in r.integers(0, 4097, size=b)]
        lens[0] = 0
        pool = [int(x) for x in r.permutation(300)[:b]] if b <= 300 else None
        run(lens, pool, t, 16, sum(lens) + 5, dtype)
    # invalid rows, then a total beyond the capacity
    run([3, -1, 5000, 2, 4, 0], [0, 1, 2, 300, 3, -2], t, 8, 100, dtype)
    run([3000, 3000], [0, 1], t, 8, 5999, dtype)


@pytest.mark.gpu
def test_metadata_empty_and_largest_batch():
    from sglang_decode.kernels.csr_metadata import csr_metadata
    t = table(4096, 8, 5)
    r = np.random.Generator(np.random.PCG64(6))
    lens = [int(x) for x in r.integers(0, 9, size=4096)]
    run(lens, [int(x) for x in r.permutation(4096)], t, 4, sum(lens))
    indptr = torch.full((2,), -9, dtype=torch.int32, device="cuda")
    e = torch.empty(0, dtype=torch.int32, device="cuda")
    csr_metadata(e, e, torch.from_numpy(t).cuda(), 4, indptr, e)
    torch.cuda.synchronize()
    assert indptr.tolist() == [0, -9]
    with pytest.raises(ValueError):  # kv_indptr shorter than batch + 1
        csr_metadata(e, e, torch.from_numpy(t).cuda(), 4, indptr[:0], e)
    with pytest.raises(ValueError):  # float lengths
        csr_metadata(e.float(), e, torch.from_numpy(t).cuda(), 4, indptr, e)


@pytest.mark.gpu
def test_metadata_feeds_plan_and_attention():
    """seq_lens -> (one launch) kv_indptr / kv_indices / splits + plan inputs -> plan ->
    attention: the outputs match the FP32 oracle over the produced metadata, and the plan
    equals the oracle plan of the harness split counts."""
    from oracle import attention as OA
    from oracle import plan as OP
    from gpu_util import assert_plan_equal, cfg_ns, close, read_plan
    from sglang_decode.config import DecodeConfig
    from sglang_decode.kernels.csr_metadata import csr_metadata
    from sglang_decode.runtime.engine import DecodeEngine
    c = DecodeConfig(batch_capacity=16, max_context=2048, workers=64, page_size=1)
    lens = [700, 0, 33, 2048, 1, 129, 1500]
    b, tokens = len(lens), 40_000
    t = table(32, 2048, 7) % tokens
    pool = [5, 0, 31, 2, 17, 9, 11]
    eng = DecodeEngine(c, kernel="valu")
    indptr = torch.zeros(b + 1, dtype=torch.int32, device="cuda")
    indices = torch.zeros(sum(lens), dtype=torch.int32, device="cuda")
    csr_metadata(torch.tensor(lens, device="cuda"), torch.tensor(pool, device="cuda"), torch.from_numpy(t).cuda(),
                 c.max_splits, indptr, indices, plan=eng.plan)
    eng.prepare()
    g = torch.Generator(device="cuda").manual_seed(8)
    q = torch.randn((c.batch_capacity, c.query_heads, c.head_dim), generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn((tokens, c.kv_heads, c.head_dim), generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn((tokens, c.kv_heads, c.head_dim), generator=g, device="cuda").to(torch.bfloat16)
    out = eng.execute(q, k, v, indices, indptr=indptr)
    torch.cuda.synchronize()
    splits = OM.harness_splits(lens, c.max_splits)
    lw, sw = lens + [0] * (c.batch_capacity - b), splits + [1] * (c.batch_capacity - b)
    assert_plan_equal(read_plan(eng.plan), OP.full_plan(lw, sw, b, cfg_ns(c)), c, b, "metadata")
    close(out[:b], OA.csr_attention(q, k, v, indptr.cpu(), indices.cpu(), lens)[:b])
