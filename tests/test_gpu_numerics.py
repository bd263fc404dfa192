"""Numerical edge cases of the attention kernels on the device, each against a closed form or
the FP32 oracle (2e-2 abs / 1e-2 rel): scores spanning hundreds of log units (the online
softmax must rescale its running state from tile to tile and split to split without
overflow), one dominant token anywhere in a row (the output is that token's V row), all
keys equal (the output is the mean of the V rows), and large V values in fp16 (fp32
accumulation, one rounding at the end).  Every kernel that takes the shape runs each case,
with several splits per request so the merge combines states of very different maxima."""
import pytest
import torch

from oracle import attention as OA
from sglang_decode import workloads as W
from sglang_decode.config import DecodeConfig, Mode
from sglang_decode.runtime.engine import DecodeEngine

from gpu_util import close

pytestmark = pytest.mark.gpu

LENGTHS = [1, 31, 200, 777, 2048, 1500]


def config(group):
    return DecodeConfig(batch_capacity=8, max_splits=8, max_context=2048, query_heads=8 * group, kv_heads=8,
                        head_dim=128, page_size=1, workers=64)


def kernels(group):
    return ["valu", "mfma", "generic"] if group <= 4 else ["mfma", "generic"]


def run(c, kernel, q, k, v, indptr, indices, lengths, dtype, scale=None):
    engine = DecodeEngine(c, dtype=dtype, force_mode=Mode.D1, kernel=kernel)
    W.update_plan(engine, lengths, W.split_hints(lengths, c.max_splits))
    engine.layers[0].partial.fill_(float("nan"))
    engine.prepare()
    out = engine.execute(q, k, v, indices, indptr=indptr, scale=scale)
    torch.cuda.synchronize()
    assert engine.last_kernel == kernel
    return out


@pytest.mark.parametrize("group", [4, 8])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_wide_score_range(group, dtype):
    """Scale 4: scores of N(0, 4 * sqrt(128)) -- a spread of ~200 log units per row."""
    c = config(group)
    q, k, v, indptr, indices = W.make_csr_inputs(c, LENGTHS, seed=5, dtype=dtype)
    expected = OA.csr_attention(q, k, v, indptr, indices, LENGTHS, scale=4.0)
    for kernel in kernels(group):
        print(f"wide scores group={group} dtype={dtype} kernel={kernel}", flush=True)
        out = run(c, kernel, q, k, v, indptr, indices, LENGTHS, dtype, scale=4.0)
        assert torch.isfinite(out[:len(LENGTHS)].float()).all(), kernel
        close(out[:len(LENGTHS)], expected[:len(LENGTHS)], msg=kernel)


@pytest.mark.parametrize("group", [4, 8])
def test_dominant_token(group):
    """Each request has one key equal to 8 x its first q head's row; every other key is
    small, so that head's output is the dominant token's V row (its weight is 1 - O(e^-40))."""
    c = config(group)
    dtype = torch.bfloat16
    q, k, v, indptr, indices = W.make_csr_inputs(c, LENGTHS, seed=6, dtype=dtype)
    k.mul_(0.01)
    ptr = indptr.cpu().tolist()
    spots = [0, 30, 199, 512, 2047, 1024]  # first, last, and tile / split boundaries
    for r, (n, t) in enumerate(zip(LENGTHS, spots)):
        t = min(t, n - 1)
        slot = int(indices[ptr[r] + t])
        for g in range(c.kv_heads):
            k[slot, g] = (q[r, g * group].float() * 8.0).to(dtype)
    for kernel in kernels(group):
        print(f"dominant token group={group} kernel={kernel}", flush=True)
        out = run(c, kernel, q, k, v, indptr, indices, LENGTHS, dtype)
        for r, (n, t) in enumerate(zip(LENGTHS, spots)):
            t = min(t, n - 1)
            slot = int(indices[ptr[r] + t])
            for g in range(c.kv_heads):
                close(out[r, g * group], v[slot, g].float().cpu().numpy(), msg=f"{kernel} request {r} kv head {g}")


@pytest.mark.parametrize("group", [4, 8])
def test_equal_keys_give_the_mean_of_v(group):
    c = config(group)
    dtype = torch.bfloat16
    q, k, v, indptr, indices = W.make_csr_inputs(c, LENGTHS, seed=7, dtype=dtype)
    k.copy_(k[:1].expand_as(k))
    ptr = indptr.cpu().tolist()
    for kernel in kernels(group):
        print(f"equal keys group={group} kernel={kernel}", flush=True)
        out = run(c, kernel, q, k, v, indptr, indices, LENGTHS, dtype)
        for r, n in enumerate(LENGTHS):
            rows = v[indices[ptr[r]:ptr[r] + n].long()].float().mean(0)  # [Hkv, D]
            expected = rows.repeat_interleave(group, 0).cpu().numpy()
            close(out[r], expected, msg=f"{kernel} request {r}")


def test_large_values_fp16():
    """V of N(0, 3000^2) in fp16 (up to ~1.3e4): the output stays finite, and within the
    unit-scale tolerance scaled by 3000 in absolute terms -- P is rounded to the KV dtype
    before P.V (kernels/attention.py:78) where the FP32 oracle keeps it exact, so the
    absolute error grows with |V| where rows cancel to near zero."""
    c = config(4)
    dtype = torch.float16
    vscale = 3000.0
    q, k, v, indptr, indices = W.make_csr_inputs(c, LENGTHS, seed=8, dtype=dtype)
    v.mul_(vscale)
    expected = OA.csr_attention(q, k, v, indptr, indices, LENGTHS)
    for kernel in kernels(4):
        print(f"large values fp16 kernel={kernel}", flush=True)
        out = run(c, kernel, q, k, v, indptr, indices, LENGTHS, dtype)
        assert torch.isfinite(out[:len(LENGTHS)].float()).all(), kernel
        close(out[:len(LENGTHS)], expected[:len(LENGTHS)], atol=2e-2 * vscale, msg=kernel)
