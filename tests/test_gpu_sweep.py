"""Seeded random sweep of decode attention against the FP32 oracle (2e-2 abs / 1e-2 rel):
each case draws its own configuration -- GQA group 1-16, head_dim 64/128/256, paged (page
sizes 2-64 and a non-power-of-two 12) or CSR, batch capacity, worker count, max_splits,
ragged lengths with empty rows and rows at max_context, per-request split counts, scale,
dtype, schedule -- and runs it on every kernel that supports the shape (the reference's
own tests fix their shapes, tests/gpu/test_decode.py; the sweep covers the combinations
between them).  Each case prints its draw first, so a failure names it."""
import numpy as np
import pytest
import torch

from oracle import attention as OA
from sglang_decode import workloads as W
from sglang_decode.config import DecodeConfig, Mode
from sglang_decode.planning.reference import split_records
from sglang_decode.runtime.engine import DecodeEngine

from gpu_util import close

pytestmark = pytest.mark.gpu

CASES = 150
WORK_BUDGET = 32_000 * 32 * 128  # sum(lengths) x Hq x D per case: keeps the oracle to ~1 s


def draw(seed):
    r = np.random.Generator(np.random.PCG64(1000 + seed))
    pick = lambda xs: xs[int(r.integers(len(xs)))]
    group, hkv = pick([1, 2, 4, 8, 16]), pick([1, 2, 4, 8])
    d = pick([64, 128, 128, 128, 128, 256])
    csr = bool(r.random() < 0.5)
    page = 1 if csr else pick([2, 4, 8, 16, 16, 32, 64, 12])
    bcap = int(r.integers(1, 41))
    n = int(r.integers(1, bcap + 1))
    max_context = pick([128, 1000, 4096, 16384])
    max_splits = pick([1, 3, 8, 16])
    workers = pick([1, 7, 64, 108, 256, 300, 512])
    kinds = r.choice(4, size=n, p=[0.1, 0.3, 0.4, 0.2])  # empty, short, medium, full
    lengths = [0 if k == 0 else int(r.integers(1, 65)) if k == 1 else
               int(r.integers(65, max_context + 1)) if k == 2 else max_context for k in kinds]
    total, budget = sum(lengths), WORK_BUDGET // (group * hkv * d)
    if total > budget:  # scale down, keeping empty rows empty and lengths within max_context
        lengths = [min(max_context, max(1, x * budget // total)) if x else 0 for x in lengths]
    splits = [int(r.integers(1, max_splits + 1)) for _ in lengths]
    c = DecodeConfig(batch_capacity=bcap, max_splits=max_splits, max_context=max_context,
                     query_heads=group * hkv, kv_heads=hkv, head_dim=d, page_size=page, workers=workers)
    dtype = pick([torch.bfloat16, torch.float16])
    mode = pick(list(Mode))
    scale = float(pick([None, 0.05, 0.3]) or d ** -0.5)
    return c, csr, lengths, splits, dtype, mode, scale


def kernels_for(c, csr):
    """The kernels whose host checks accept the shape (csrc/attention.hip select_kernel): the
    MFMA kernel (groups <= 16) and the VALU kernel (groups <= 4) take head_dim 64, 128 and 256
    and any page size (a power of two by shift and mask, any other by division)."""
    ks = ["generic", "mfma"]
    if c.group_size <= 4:
        ks.append("valu")
    return ks


@pytest.mark.parametrize("seed", range(CASES))
def test_random_configuration(seed):
    c, csr, lengths, splits, dtype, mode, scale = draw(seed)
    print(f"seed {seed}: {c} csr={csr} dtype={dtype} mode={mode.name} lengths={lengths} splits={splits}",
          flush=True)
    if csr:
        q, k, v, indptr, indices = W.make_csr_inputs(c, lengths, seed=seed, dtype=dtype)
        expected = OA.csr_attention(q, k, v, indptr, indices, lengths, scale=scale)
        inputs = (q, k, v, indices)
    else:
        q, k, v, pages = W.make_inputs(c, lengths, seed=seed, dtype=dtype)
        expected = OA.paged_attention(q, k, v, pages, lengths, c.page_size, scale=scale)
        inputs, indptr = (q, k, v, pages), None
    n = len(lengths)
    records, counts, _ = split_records(lengths, splits, c)
    for kernel in kernels_for(c, csr):
        print(f"seed {seed}: kernel {kernel}", flush=True)
        engine = DecodeEngine(c, dtype=dtype, force_mode=mode, kernel=kernel)
        W.update_plan(engine, lengths, splits)
        engine.layers[0].partial.fill_(float("nan"))
        engine.layers[0].lse.fill_(float("nan"))
        engine.prepare()
        out = engine.execute(*inputs, indptr=indptr, scale=scale)
        torch.cuda.synchronize()
        assert engine.last_kernel == kernel
        assert engine.plan.error.item() == 0, kernel
        assert engine.plan.record_count.item() == len(records), kernel
        assert engine.plan.counts[:n].tolist() == counts, kernel
        close(out[:n], expected[:n], msg=f"seed {seed} kernel {kernel}")
        assert not out[n:].float().abs().sum().item(), kernel  # rows past the batch stay zero
