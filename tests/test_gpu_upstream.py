"""The upstream two-stage split-KV comparator (sgd_upstream_decode, the reference's
benchmarks/baselines.py:8-34 over third_party/sglang/decode_attention.py:245-601) against
the FP32 oracle: outputs within 2e-2 abs / 1e-2 rel, and every non-empty split slot equal
to the oracle's split partial / LSE -- its splits are the plan's records (the same
ceil(ceil(L/S)/32)*32 chunking), so the persistent path's slots must agree with it too."""
import numpy as np
import pytest
import torch

from oracle import attention as OA
from sglang_decode import workloads as W
from sglang_decode.config import DecodeConfig, Mode
from sglang_decode.kernels.upstream import decode_attention_fwd
from sglang_decode.planning.reference import split_records
from sglang_decode.runtime.engine import DecodeEngine

from gpu_util import close

pytestmark = pytest.mark.gpu


def _run(c, lengths, splits, dtype, seed):
    q, k, v, indptr, indices = W.make_csr_inputs(c, lengths, seed=seed, dtype=dtype, pool_tokens=1 << 16)
    b = len(lengths)
    logits = torch.full((b, c.query_heads, c.max_splits, c.head_dim), float("nan"), device="cuda")
    lse = torch.full((b, c.query_heads, c.max_splits), float("nan"), device="cuda")
    out = torch.empty((b, c.query_heads, c.head_dim), dtype=dtype, device="cuda")
    num = torch.tensor(splits, dtype=torch.int32, device="cuda")
    decode_attention_fwd(q[:b], k, v, out, indptr[:b + 1].contiguous(), indices, logits, lse, num, c.max_splits,
                         c.head_dim ** -0.5)
    torch.cuda.synchronize()
    return q, k, v, indptr, indices, out, logits, lse


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("lengths,smax", [([0, 1, 17, 33, 257, 513, 4000], 16), ([64] * 9, 1), ([8192, 3, 900], 64)])
def test_upstream_matches_oracle_and_split_slots(lengths, smax, dtype):
    c = DecodeConfig(batch_capacity=len(lengths), max_splits=smax, max_context=8192, page_size=1, workers=64)
    splits = W.split_hints(lengths, smax)
    print(f"upstream lengths={lengths} smax={smax} dtype={dtype}", flush=True)
    q, k, v, indptr, indices, out, logits, lse = _run(c, lengths, splits, dtype, seed=len(lengths))
    close(out, OA.csr_attention(q, k, v, indptr, indices, lengths)[:len(lengths)])
    records, _, _ = split_records(lengths, splits, c)
    maxl = max(max(lengths), 1)
    table = torch.zeros((len(lengths), maxl), dtype=torch.int32)
    for r, n in enumerate(lengths):
        table[r, :n] = indices[int(indptr[r]):int(indptr[r]) + n].cpu()
    ref = OA.split_partials(q, k[:, None], v[:, None], table, lengths, 1,
                            [(x.request, x.split, x.begin, x.end) for x in records], c.query_heads, c.max_splits)
    lo, ls = logits.cpu().numpy(), lse.cpu().numpy()
    close(np.stack([lo[r, h, s] for (r, h, s) in ref]), np.stack([x[0] for x in ref.values()]))
    close(np.array([ls[r, h, s] for (r, h, s) in ref]), np.array([x[1] for x in ref.values()]), atol=1e-2, rtol=1e-3)


def test_upstream_agrees_with_persistent_path_on_llama8b_batch64():
    """The batch-64 Llama-3-8B layer: the comparator and the persistent D1 engine on the
    same inputs both match the oracle (every request)."""
    c = W.config_for("c2")
    lengths = W.c2_lengths()
    splits = W.split_hints(lengths, c.max_splits)
    q, k, v, indptr, indices = W.make_csr_inputs(c, lengths, seed=88, pool_tokens=1 << 20)
    b = len(lengths)
    logits = torch.empty((b, c.query_heads, c.max_splits, c.head_dim), device="cuda")
    lse = torch.empty((b, c.query_heads, c.max_splits), device="cuda")
    out = torch.empty((b, c.query_heads, c.head_dim), dtype=torch.bfloat16, device="cuda")
    num = torch.tensor(splits, dtype=torch.int32, device="cuda")
    decode_attention_fwd(q[:b], k, v, out, indptr, indices, logits, lse, num, c.max_splits, c.head_dim ** -0.5)
    engine = DecodeEngine(c, force_mode=Mode.D1)
    W.update_plan(engine, lengths, splits)
    engine.prepare()
    mine = engine.execute(q, k, v, indices, indptr=indptr)
    torch.cuda.synchronize()
    rows = indices.long()
    host = (q.cpu(), k[rows].cpu(), v[rows].cpu(), indptr.cpu(), torch.arange(rows.numel(), dtype=torch.int32))
    expected = OA.csr_attention(*host, lengths)
    close(out, expected[:b])
    close(mine[:b], expected[:b])
