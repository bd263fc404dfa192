"""sgd_decode_noalloc (no device allocation: plan tables, counters and split slots in the
library's static device array) against the allocating entry points it stands for --
sgd_build_plan + sgd_persistent_decode + sgd_merge_splits through DecodeEngine -- on
two calls in a row, the second with a smaller batch and shorter contexts.  Same kernels,
same plan: the outputs must be bitwise equal, and within 2e-2 abs / 1e-2 rel of the FP32
oracle."""
import pytest
import torch

from oracle import attention as OA
from sglang_decode import workloads as W
from sglang_decode.config import DecodeConfig, Mode
from sglang_decode.kernels.noalloc import decode_noalloc
from sglang_decode.runtime.engine import DecodeEngine

from gpu_util import close

pytestmark = pytest.mark.gpu


def _plan_inputs(c, lengths, splits):
    dev = torch.device("cuda", torch.cuda.current_device())
    L = torch.zeros(c.batch_capacity, dtype=torch.int32)
    S = torch.ones(c.batch_capacity, dtype=torch.int32)
    L[:len(lengths)] = torch.tensor(lengths, dtype=torch.int32)
    S[:len(splits)] = torch.tensor(splits, dtype=torch.int32)
    return L.to(dev), S.to(dev), torch.tensor([len(lengths)], dtype=torch.int32, device=dev)


def _allocating(c, mode, lengths, splits, inputs, indptr, dtype):
    engine = DecodeEngine(c, dtype=dtype, force_mode=mode)
    W.update_plan(engine, lengths, splits)
    engine.prepare()
    return engine.execute(*inputs, indptr=indptr).clone()


@pytest.mark.parametrize("mode", [Mode.D1, Mode.R1, Mode.STATIC])
def test_noalloc_matches_allocating_entry_csr_llama8b(mode):
    c = W.config_for("c2")
    out = torch.full((c.batch_capacity, c.query_heads, c.head_dim), float("nan"), dtype=torch.bfloat16,
                     device="cuda")
    full = W.c2_lengths()
    for n, shrink in ((24, 1), (9, 3)):  # the second call: fewer rows, shorter contexts
        lengths = [max(1, x // shrink) for x in full[:n]]
        splits = W.split_hints(lengths, c.max_splits)
        print(f"noalloc csr mode={mode.name} batch={n} total={sum(lengths)}", flush=True)
        q, k, v, indptr, indices = W.make_csr_inputs(c, lengths, seed=70 + n, pool_tokens=1 << 16)
        expect = _allocating(c, mode, lengths, splits, (q, k, v, indices), indptr, torch.bfloat16)
        L, S, A = _plan_inputs(c, lengths, splits)
        got = decode_noalloc(c, q, k, v, indices, L, S, A, out, indptr=indptr, force_mode=mode)
        torch.cuda.synchronize()
        assert torch.equal(got, expect)
        close(got[:n], OA.csr_attention(q, k, v, indptr, indices, lengths)[:n])
        assert not got[n:].float().abs().sum().item()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_noalloc_matches_allocating_entry_paged_group8(dtype):
    c = DecodeConfig(batch_capacity=8, max_splits=8, max_context=4096, query_heads=64, kv_heads=8,
                     page_size=16, workers=128)
    out = torch.empty((c.batch_capacity, c.query_heads, c.head_dim), dtype=dtype, device="cuda")
    for lengths in ([4096, 1, 999, 64, 0, 2500, 31, 700], [300, 17, 2]):
        splits = W.split_hints(lengths, c.max_splits)
        print(f"noalloc paged dtype={dtype} lengths={lengths}", flush=True)
        q, k, v, pages = W.make_inputs(c, lengths, seed=len(lengths), dtype=dtype)
        expect = _allocating(c, Mode.D4, lengths, splits, (q, k, v, pages), None, dtype)
        L, S, A = _plan_inputs(c, lengths, splits)
        got = decode_noalloc(c, q, k, v, pages, L, S, A, out, force_mode=Mode.D4)
        torch.cuda.synchronize()
        assert torch.equal(got, expect)
        n = len(lengths)
        close(got[:n], OA.paged_attention(q, k, v, pages, lengths, c.page_size)[:n])


def test_noalloc_invalid_metadata_writes_nan():
    c = DecodeConfig(batch_capacity=4, max_context=512, workers=32)
    q, k, v, pages = W.make_inputs(c, [100, 512])
    out = torch.zeros((c.batch_capacity, c.query_heads, c.head_dim), dtype=torch.bfloat16, device="cuda")
    L, S, A = _plan_inputs(c, [100, 600], [1, 1])  # 600 > max_context
    decode_noalloc(c, q, k, v, pages, L, S, A, out)
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()


@pytest.mark.parametrize("mode", [Mode.D4, Mode.R1])
def test_noalloc_single_split_rows_from_the_attention(mode):
    """Batch capacity 128 x 32 query heads = 4096 merge rows (16.8 MB of split slots):
    beyond one residency round of the merge on 256 CUs, so both entries let each
    request's first split write its rows and merge only the multi-split ones.  The output
    is poisoned, the second call is smaller: every row of both calls must be rewritten."""
    c = DecodeConfig(batch_capacity=128, max_splits=8, max_context=4096, page_size=1, workers=256)
    if not DecodeEngine(c).direct_first_split:
        pytest.skip("this device holds all 4096 merge rows in one residency round")
    out = torch.empty((c.batch_capacity, c.query_heads, c.head_dim), dtype=torch.bfloat16, device="cuda")
    full = W.lognormal_lengths(128, 384, 16, 3000, seed=33)
    for n, shrink in ((128, 1), (41, 2)):
        lengths = [max(1, x // shrink) for x in full[:n]]
        splits = W.split_hints(lengths, c.max_splits)
        assert 1 in splits and max(splits) > 1
        print(f"noalloc direct mode={mode.name} batch={n} single={splits.count(1)}", flush=True)
        q, k, v, indptr, indices = W.make_csr_inputs(c, lengths, seed=80 + n, pool_tokens=1 << 17)
        expect = _allocating(c, mode, lengths, splits, (q, k, v, indices), indptr, torch.bfloat16)
        L, S, A = _plan_inputs(c, lengths, splits)
        out.fill_(float("nan"))
        got = decode_noalloc(c, q, k, v, indices, L, S, A, out, indptr=indptr, force_mode=mode)
        torch.cuda.synchronize()
        assert torch.equal(got, expect)
        close(got[:n], OA.csr_attention(q, k, v, indptr, indices, lengths)[:n])
        assert not got[n:].float().abs().sum().item()
