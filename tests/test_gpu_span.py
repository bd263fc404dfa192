"""The span schedule (SGD_KERNEL_SPAN) on the GPU: its plan tables bit-exact against
the oracle's brute-force enumeration of the tile sequence, and its outputs and
per-split slots against the FP32 oracle (2e-2 abs / 1e-2 rel), including tasks cut
across many workers, more workers than tiles, and rows without context."""
import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import plan as OP
from sglang_decode import workloads as W
from sglang_decode.config import DecodeConfig, Mode
from sglang_decode.planning.reference import split_records
from sglang_decode.runtime.engine import DecodeEngine

from gpu_util import cfg_ns, close

pytestmark = pytest.mark.gpu


def run(engine, lengths, inputs, indptr=None, splits=None):
    W.update_plan(engine, lengths, splits)
    for layer in engine.layers:
        layer.partial.fill_(float("nan"))
        layer.lse.fill_(float("nan"))
        layer.edge.fill_(float("nan"))
    engine.prepare()
    q, k, v, pages = inputs
    out = engine.execute(q, k, v, pages, indptr=indptr)
    torch.cuda.synchronize()
    assert engine.attention_kernel_name() == "span"
    return out


def csr_case(c, lengths, seed, splits=None, mode=Mode.R1, dtype=torch.bfloat16):
    q, k, v, indptr, indices = W.make_csr_inputs(c, lengths, seed=seed, dtype=dtype)
    engine = DecodeEngine(c, dtype=dtype, force_mode=mode, kernel="span")
    out = run(engine, lengths, (q, k, v, indices), indptr=indptr, splits=splits)
    n = len(lengths)
    close(out[:n], OA.csr_attention(q, k, v, indptr, indices, lengths)[:n])
    assert not out[n:].float().abs().sum().item()
    return engine, (q, k, v, indptr, indices)


@pytest.mark.parametrize("mode", [Mode.R0, Mode.R1, Mode.D4])
@pytest.mark.parametrize("lengths,splits", [
    ([0, 1, 33, 513], [16, 16, 16, 2]),
    ([300, 0, 0, 17, 4096, 1, 0, 2000], None),
    ([1], None),
])
def test_span_tables_match_oracle(mode, lengths, splits):
    c = DecodeConfig(batch_capacity=8, max_context=4096, page_size=1)
    splits = splits or W.split_hints(lengths, c.max_splits)
    engine = DecodeEngine(c, force_mode=mode, kernel="span")
    W.update_plan(engine, lengths, splits)
    engine.prepare()
    torch.cuda.synchronize()
    ns = cfg_ns(c)
    ns.span_units = engine.plan.span_units
    ref = OP.span_tables(lengths, splits, len(lengths), ns)
    assert engine.plan.tile_prefix.tolist() == ref["tile_prefix"]
    assert engine.plan.span.tolist() == ref["span"]


@pytest.mark.parametrize("mode", [Mode.R0, Mode.R1, Mode.STATIC, Mode.D1, Mode.D4])
def test_span_llama8b_shape_every_mode(mode):
    c = W.config_for("c2")
    csr_case(c, W.c2_lengths()[:24], seed=9, mode=mode)


@pytest.mark.parametrize("splits", [[1], [16]])
def test_span_one_long_request(splits):
    """One 32768-token request: with one split its task per kv head is 2048 tiles, so
    each is cut across ~32 workers and completed from their edge states."""
    c = DecodeConfig(batch_capacity=2, max_splits=16, max_context=32768, page_size=1, workers=256)
    csr_case(c, [32768], seed=4, splits=splits)


def test_span_more_workers_than_tiles():
    c = DecodeConfig(batch_capacity=4, max_context=256, page_size=1, workers=512)
    csr_case(c, [1, 3], seed=6)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_span_rows_without_context_and_fp16(dtype):
    c = DecodeConfig(batch_capacity=16, max_context=8192, page_size=1, workers=256)
    csr_case(c, [0, 700, 0, 0, 5, 8192, 0, 129, 1, 0], seed=8, dtype=dtype, mode=Mode.D1)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_span_paged(dtype):
    c = DecodeConfig(batch_capacity=8, max_context=4096, workers=256)  # page 16
    lengths = [4096, 1, 17, 1000, 2047]
    inputs = W.make_inputs(c, lengths, seed=21, dtype=dtype)
    engine = DecodeEngine(c, dtype=dtype, force_mode=Mode.D4, kernel="span")
    out = run(engine, lengths, inputs)
    close(out[:5], OA.paged_attention(*inputs[:3], inputs[3], lengths, c.page_size)[:5])


def test_span_split_slots_match_oracle():
    """After execute every (request, head, split) slot holds that split's normalized
    partial and LSE -- tasks cut across workers included (written by the merge)."""
    c = DecodeConfig(batch_capacity=8, max_context=2048, workers=64)
    lengths = [700, 5, 129, 2048, 1, 300]
    splits = [3, 1, 2, 16, 1, 4]
    inputs = W.make_inputs(c, lengths, seed=3)
    engine = DecodeEngine(c, force_mode=Mode.R1, kernel="span")
    run(engine, lengths, inputs, splits=splits)
    records, _, _ = split_records(lengths, splits, c)
    ref = OA.split_partials(*inputs[:3], inputs[3], lengths, c.page_size,
                            [(r.request, r.split, r.begin, r.end) for r in records],
                            c.query_heads, c.max_splits)
    partial = engine.layers[0].partial.cpu().numpy()
    lse = engine.layers[0].lse.cpu().numpy()
    close(np.stack([partial[r, h, s] for (r, h, s) in ref]), np.stack([v[0] for v in ref.values()]))
    close(np.array([lse[r, h, s] for (r, h, s) in ref]), np.array([v[1] for v in ref.values()]),
          atol=1e-2, rtol=1e-3)


def test_span_repeatable():
    """The span schedule merges in a fixed order: repeated launches agree bitwise."""
    c = W.config_for("c2")
    engine, (q, k, v, indptr, indices) = csr_case(c, W.c2_lengths()[:32], seed=12)
    first = engine.layers[0].output.clone()
    for _ in range(3):
        engine.prepare()
        out = engine.execute(q, k, v, indices, indptr=indptr)
        torch.cuda.synchronize()
        assert torch.equal(out, first)
