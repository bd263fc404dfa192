"""Decode-attention parity on the GPU against the FP32 oracle (2e-2 abs / 1e-2 rel),
for every schedule, both KV layouts (paged, CSR), strides, dtypes and group sizes,
plus the per-split partial/LSE slots and the invalid-metadata path."""
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

_CACHE = {}


def paged_inputs(c, lengths, seed=17, dtype=torch.bfloat16):
    key = ("paged", c, tuple(lengths), seed, dtype)
    if key not in _CACHE:
        _CACHE.clear()
        _CACHE[key] = W.make_inputs(c, lengths, seed=seed, dtype=dtype)
    return _CACHE[key]


def run(engine, lengths, inputs, indptr=None, splits=None, scale=None):
    W.update_plan(engine, lengths, splits)
    for layer in engine.layers:
        layer.partial.fill_(float("nan"))
        layer.lse.fill_(float("nan"))
    engine.prepare()
    q, k, v, pages = inputs
    out = engine.execute(q, k, v, pages, indptr=indptr, scale=scale)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("kernel", ["auto", "generic", "valu", "mfma"])
@pytest.mark.parametrize("mode", list(Mode))
@pytest.mark.parametrize("lengths", [[0, 1, 17, 33, 257, 513], [256] * 24 + [1536] * 4 + [16384] * 4])
def test_outputs_and_plan_every_mode(mode, lengths, kernel):
    c = DecodeConfig()  # reference defaults: page 16, Bcap 64, Hq/Hkv 32/8, D 128, 108 workers
    engine = DecodeEngine(c, force_mode=mode, kernel=kernel)
    inputs = paged_inputs(c, lengths)
    out = run(engine, lengths, inputs)
    expected = OA.paged_attention(*inputs[:3], inputs[3], lengths, c.page_size)
    n = len(lengths)
    close(out[:n], expected[:n])
    assert not out[n:].float().abs().sum().item()  # inactive rows are exact zeros
    assert engine.plan.error.item() == 0
    records, counts, _ = split_records(lengths, W.split_hints(lengths), c)
    assert engine.plan.record_count.item() == len(records)
    assert engine.plan.counts[:n].tolist() == counts


def test_partial_and_lse_slots_match_oracle():
    c = DecodeConfig(batch_capacity=8, max_context=2048, workers=64)
    lengths = [700, 5, 129, 2048, 1, 300]
    splits = [3, 1, 2, 16, 1, 4]
    inputs = paged_inputs(c, lengths, seed=3)
    engine = DecodeEngine(c, force_mode=Mode.D4)
    run(engine, lengths, inputs, splits=splits)
    records, _, _ = split_records(lengths, splits, c)
    ref = OA.split_partials(*inputs[:3], inputs[3], lengths, c.page_size,
                            [(r.request, r.split, r.begin, r.end) for r in records],
                            c.query_heads, c.max_splits)
    partial = engine.layers[0].partial.cpu().numpy()
    lse = engine.layers[0].lse.cpu().numpy()
    got_p = np.stack([partial[r, h, s] for (r, h, s) in ref])
    got_l = np.array([lse[r, h, s] for (r, h, s) in ref])
    close(got_p, np.stack([v[0] for v in ref.values()]))
    close(got_l, np.array([v[1] for v in ref.values()]), atol=1e-2, rtol=1e-3)


@pytest.mark.parametrize("mode", [Mode.R1, Mode.STATIC, Mode.D1])
def test_csr_small_config(mode):
    c = W.config_for("c1")
    lengths = W.c1_lengths()
    q, k, v, indptr, indices = W.make_csr_inputs(c, lengths, seed=5, pool_tokens=4096)
    engine = DecodeEngine(c, force_mode=mode)
    out = run(engine, lengths, (q, k, v, indices), indptr=indptr)
    close(out[:len(lengths)], OA.csr_attention(q, k, v, indptr, indices, lengths)[:len(lengths)])


@pytest.mark.parametrize("kernel", ["valu", "mfma"])
@pytest.mark.parametrize("mode", [Mode.R1, Mode.STATIC, Mode.D1, Mode.D4, Mode.R0])
def test_csr_llama8b_shape(mode, kernel):
    c = W.config_for("c2")
    lengths = W.c2_lengths()[:16]
    q, k, v, indptr, indices = W.make_csr_inputs(c, lengths, seed=9, pool_tokens=1 << 16)
    engine = DecodeEngine(c, force_mode=mode, kernel=kernel)
    out = run(engine, lengths, (q, k, v, indices), indptr=indptr)
    close(out[:16], OA.csr_attention(q, k, v, indptr, indices, lengths)[:16])


def test_noncontiguous_kv_strides():
    c = DecodeConfig()
    lengths = [17, 513]
    q, k, v, pages = W.make_inputs(c, lengths)

    def strided(x):
        storage = torch.empty((*x.shape[:-1], x.shape[-1] * 2), device=x.device, dtype=x.dtype)
        storage[..., ::2].copy_(x)
        return storage[..., ::2]

    ks, vs = strided(k), strided(v)
    engine = DecodeEngine(c, force_mode=Mode.D4)
    out = run(engine, lengths, (q, ks, vs, pages))
    close(out[:2], OA.paged_attention(q, k, v, pages, lengths, c.page_size)[:2])
    # a transposed (non-contiguous) page table
    table = pages.t().contiguous().t()
    out = run(engine, lengths, (q, k, v, table))
    close(out[:2], OA.paged_attention(q, k, v, pages, lengths, c.page_size)[:2])


@pytest.mark.parametrize("hq,kernel", [(32, "valu"), (32, "mfma"), (32, "generic"), (64, "mfma"), (64, "generic")])
def test_views_of_packed_projection_and_fused_kv(hq, kernel):
    """q as heads of a packed [B, (Hq + 2 Hkv) D] projection and CSR K/V as halves of one
    [tokens, 2, Hkv, D] buffer: row strides that are not Hq D / Hkv D, unit dim strides, so
    the tuned kernels take them (sglang_backend.py:102-103 hands the kernel such views)."""
    c = DecodeConfig(batch_capacity=8, max_splits=8, max_context=2048, query_heads=hq, kv_heads=8, page_size=1,
                     workers=64)
    lengths = [1, 100, 2048, 517, 0, 64]
    q0, k0, v0, indptr, indices = W.make_csr_inputs(c, lengths, seed=31)
    b, d, hkv = c.batch_capacity, c.head_dim, c.kv_heads
    qkv = torch.randn((b, (hq + 2 * hkv) * d), device="cuda", dtype=q0.dtype)
    qkv[:, :hq * d] = q0.reshape(b, hq * d)
    q = qkv[:, :hq * d].view(b, hq, d)
    kv = torch.empty((k0.shape[0], 2, hkv, d), device="cuda", dtype=k0.dtype)
    kv[:, 0].copy_(k0)
    kv[:, 1].copy_(v0)
    k, v = kv[:, 0], kv[:, 1]
    assert not q.is_contiguous() and not k.is_contiguous() and k.stride(2) == 1
    engine = DecodeEngine(c, force_mode=Mode.D1, kernel=kernel)
    out = run(engine, lengths, (q, k, v, indices), indptr=indptr)
    assert engine.last_kernel == kernel
    n = len(lengths)
    close(out[:n], OA.csr_attention(q0, k0, v0, indptr, indices, lengths)[:n])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hq,hkv,d", [(8, 8, 128), (16, 8, 128), (64, 8, 128), (32, 2, 128),
                                      (16, 4, 64), (16, 4, 256)])
def test_group_sizes_dims_dtypes(hq, hkv, d, dtype):
    c = DecodeConfig(batch_capacity=6, max_context=4096, query_heads=hq, kv_heads=hkv, head_dim=d,
                     page_size=16, workers=96)
    lengths = [4096, 1, 999, 64, 0, 2500]
    inputs = W.make_inputs(c, lengths, seed=11, dtype=dtype)
    engine = DecodeEngine(c, dtype=dtype, force_mode=Mode.D1)
    out = run(engine, lengths, inputs, scale=0.07)
    close(out[:6], OA.paged_attention(*inputs[:3], inputs[3], lengths, c.page_size, scale=0.07))


def test_invalid_metadata_writes_nan_and_schedules_nothing():
    c = DecodeConfig(batch_capacity=4, max_context=512, workers=32)
    lengths = [100, 600]  # 600 > max_context
    inputs = W.make_inputs(c, [100, 512])
    engine = DecodeEngine(c)
    out = run(engine, lengths, inputs, splits=[1, 1])
    assert engine.plan.error.item() == 1 and engine.plan.record_count.item() == 0
    assert torch.isnan(out.float()).all()


@pytest.mark.parametrize("kernel", ["auto", "valu", "mfma"])
def test_reused_output_buffer_and_repeated_execute(kernel):
    c = W.config_for("c1")
    lengths = [200, 16, 100, 50]
    q, k, v, indptr, indices = W.make_csr_inputs(c, lengths, seed=21)
    engine = DecodeEngine(c, force_mode=Mode.D4, kernel=kernel)
    out1 = run(engine, lengths, (q, k, v, indices), indptr=indptr).clone()
    out2 = engine.execute(q, k, v, indices, indptr=indptr)  # same plan, second execute
    torch.cuda.synchronize()
    assert out2.data_ptr() == engine.layers[0].output.data_ptr()
    assert torch.equal(out1, out2)  # fixed merge order: bitwise repeatable


@pytest.mark.parametrize("workers", [256, 108, 37])
def test_auto_kernel_is_bitwise_repeatable_at_any_worker_count(workers):
    """AUTO with one worker per CU (the reference's convention, sglang_backend.py:42),
    DecodeConfig's default 108 and an odd count: every launch merges in a fixed order,
    so repeated dynamic-claim launches give identical bits."""
    c = W.config_for("c2", workers=workers)
    lengths = W.c2_lengths()[:24]
    q, k, v, indptr, indices = W.make_csr_inputs(c, lengths, seed=23, pool_tokens=1 << 16)
    engine = DecodeEngine(c, force_mode=Mode.D1)
    first = run(engine, lengths, (q, k, v, indices), indptr=indptr).clone()
    for _ in range(3):
        again = engine.execute(q, k, v, indices, indptr=indptr)
        torch.cuda.synchronize()
        assert torch.equal(first, again)
    assert engine.attention_kernel_name() == "valu"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("mode", list(Mode))
@pytest.mark.parametrize("hq", [8, 32, 64, 128])
def test_mfma_kernel_groups_paged(hq, mode, dtype):
    """Groups 1, 4, 8 (Llama-3-70B heads) and 16 on the MFMA kernel (heads padded to 16):
    page 16, ragged lengths (a 1-token request, a 31-token one that ends mid-tile, an
    empty row)."""
    c = DecodeConfig(batch_capacity=6, max_splits=16, max_context=4096, query_heads=hq, kv_heads=8,
                     head_dim=128, page_size=16, workers=64)
    lengths = [4096, 1, 999, 31, 0, 2500]
    inputs = W.make_inputs(c, lengths, seed=23, dtype=dtype)
    engine = DecodeEngine(c, dtype=dtype, force_mode=mode, kernel="mfma")
    out = run(engine, lengths, inputs, scale=0.07)
    assert engine.attention_kernel_name() == "mfma"
    close(out[:6], OA.paged_attention(*inputs[:3], inputs[3], lengths, c.page_size, scale=0.07))


@pytest.mark.parametrize("mode", [Mode.R1, Mode.D1, Mode.STATIC])
def test_mfma_kernel_csr(mode):
    c = DecodeConfig(batch_capacity=8, max_splits=8, max_context=3000, query_heads=64, kv_heads=8,
                     head_dim=128, page_size=1, workers=40)
    lengths = [3000, 17, 640, 1, 2049, 0, 33, 700]
    q, k, v, indptr, indices = W.make_csr_inputs(c, lengths, seed=29, pool_tokens=1 << 14)
    engine = DecodeEngine(c, force_mode=mode)  # auto picks the MFMA kernel for group 8
    out = run(engine, lengths, (q, k, v, indices), indptr=indptr)
    assert engine.attention_kernel_name() == "mfma"
    close(out[:8], OA.csr_attention(q, k, v, indptr, indices, lengths)[:8])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_llama70b_paged_shape_subset(dtype):
    """The 70B paged configuration (page 16, 64 q / 8 kv, contexts in [2048, 16384]) on
    the first 6 of its seeded requests."""
    full = W.config_for("c4")
    c = DecodeConfig(batch_capacity=6, max_splits=full.max_splits, max_context=full.max_context,
                     query_heads=64, kv_heads=8, head_dim=128, page_size=16, workers=128)
    lengths = W.c4_lengths()[:6]
    inputs = W.make_inputs(c, lengths, seed=41, dtype=dtype)
    engine = DecodeEngine(c, dtype=dtype, force_mode=Mode.D1)
    out = run(engine, lengths, inputs)
    close(out[:6], OA.paged_attention(*inputs[:3], inputs[3], lengths, c.page_size))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("csr", [False, True])
def test_rows_with_many_splits(csr, dtype):
    """Rows of 17, 40 and 64 splits (merged by several waves of one workgroup, split
    ranges combined in a fixed order) beside rows of 1-16 splits and an empty row."""
    c = DecodeConfig(batch_capacity=8, max_splits=64, max_context=8192, page_size=1 if csr else 16, workers=64)
    lengths = [8192, 1, 2100, 0, 5000, 700, 64 * 32 + 5, 300]
    splits = [64, 1, 17, 1, 40, 16, 64, 3]
    if csr:
        q, k, v, indptr, indices = W.make_csr_inputs(c, lengths, seed=31, dtype=dtype, pool_tokens=1 << 15)
        inputs, exp = (q, k, v, indices), OA.csr_attention(q, k, v, indptr, indices, lengths)
    else:
        inputs, indptr = W.make_inputs(c, lengths, seed=31, dtype=dtype), None
        exp = OA.paged_attention(*inputs[:3], inputs[3], lengths, c.page_size)
    engine = DecodeEngine(c, dtype=dtype, force_mode=Mode.D1)
    out = run(engine, lengths, inputs, indptr=indptr, splits=splits)
    counts = engine.plan.counts[:len(lengths)].tolist()
    assert max(counts) == 64 and sum(n > 16 for n in counts) == 4  # the multi-wave path runs
    close(out[:len(lengths)], exp[:len(lengths)])
    assert not out[len(lengths):].float().abs().sum().item()


@pytest.mark.parametrize("head_dim", [64, 128, 256])
def test_merge_splits_min_rows_and_grid(head_dim):
    """sgd_merge_splits_min at the C ABI on synthetic split slots: rows of requests with 1 <=
    n < min_splits are left as they were, every other row is bitwise what sgd_merge_splits
    writes (rows of 0 splits: zeros), and a plan error writes NaN everywhere.  The batch's
    rows (256 x 32) exceed one residency round, so the kernel strides; its rows mix 0, 1,
    2, 16, 17 and 64 splits."""
    from sglang_decode import _lib
    from sglang_decode._lib import ptr
    lib = _lib.lib()
    bcap, hq, smax, d = 256, 32, 64, head_dim
    g = torch.Generator().manual_seed(7)
    counts = torch.tensor([(0, 1, 2, 16, 17, 64, 1, 1)[r % 8] for r in range(bcap)], dtype=torch.int32)
    partial = torch.randn(bcap, hq, smax, d, generator=g).cuda()
    lse = (torch.randn(bcap, hq, smax, generator=g) * 3).cuda()
    counts_d, active = counts.cuda(), torch.tensor([bcap], dtype=torch.int32).cuda()
    stream = _lib.stream_handle(partial.device)

    def merge(min_splits, error):
        out = torch.full((bcap, hq, d), 7.0, dtype=torch.bfloat16, device="cuda")
        err = torch.tensor([error], dtype=torch.int32).cuda()
        args = (ptr(partial), ptr(lse), ptr(counts_d), ptr(active), ptr(err), ptr(out), bcap, hq, d, smax)
        if min_splits is None:
            rc = lib.sgd_merge_splits(*args, _lib.SGD_BF16, stream)
        else:
            rc = lib.sgd_merge_splits_min(*args, min_splits, _lib.SGD_BF16, stream)
        assert rc == 0
        torch.cuda.synchronize()
        return out

    full = merge(None, 0)
    for m in (1, 2, 17, 65):
        part = merge(m, 0)
        skipped = (counts >= 1) & (counts < m)
        assert torch.equal(part[~skipped].view(torch.int16), full[~skipped].view(torch.int16)), m
        assert (part[skipped].float() == 7.0).all(), m
    assert not full[counts == 0].float().abs().sum().item()
    assert torch.isnan(merge(2, 1).float()).all()
    assert torch.equal(merge(1, 0).view(torch.int16), full.view(torch.int16))


def test_two_engines_on_two_streams():
    """Separate engines may run at once (runtime/engine.py:35-37): a CSR group-4 engine and a
    paged group-8 engine launched alternately on two streams, five rounds without a host
    sync in between, each output against the oracle and every claim counter back at zero."""
    c1 = DecodeConfig(batch_capacity=16, max_splits=8, max_context=4096, page_size=1, workers=512)
    c2 = DecodeConfig(batch_capacity=8, max_splits=8, max_context=4096, query_heads=64, kv_heads=8, page_size=16,
                      workers=512)
    l1 = [4096, 1, 700, 2000, 33, 4000, 129, 3000]
    l2 = [4096, 17, 1500, 999, 2048, 3]
    q1, k1, v1, indptr, indices = W.make_csr_inputs(c1, l1, seed=41)
    x2 = W.make_inputs(c2, l2, seed=42)
    e1 = DecodeEngine(c1, force_mode=Mode.D1)
    e2 = DecodeEngine(c2, force_mode=Mode.D4)
    for e, lengths in ((e1, l1), (e2, l2)):
        W.update_plan(e, lengths)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    outs = []
    for _ in range(5):
        with torch.cuda.stream(s1):
            e1.prepare()
            outs.append((0, e1.execute(q1, k1, v1, indices, indptr=indptr).clone()))
        with torch.cuda.stream(s2):
            e2.prepare()
            outs.append((1, e2.execute(*x2).clone()))
    torch.cuda.synchronize()
    exp1 = OA.csr_attention(q1, k1, v1, indptr, indices, l1)
    exp2 = OA.paged_attention(*x2[:3], x2[3], l2, c2.page_size)
    for which, out in outs:
        if which == 0:
            close(out[:len(l1)], exp1[:len(l1)], msg="csr engine")
        else:
            close(out[:len(l2)], exp2[:len(l2)], msg="paged engine")
    for e in (e1, e2):
        assert not e.sync.any().item()  # claim / finished counters back at zero


@pytest.mark.parametrize("page", [3, 12, 48])
@pytest.mark.parametrize("hq", [32, 64])
def test_page_sizes_not_a_power_of_two(page, hq):
    """Pages of 3, 12 and 48 tokens on the tuned kernels (tokens mapped to (page, row) by
    division) and the generic one, group 4 and 8, tasks and tiles crossing page ends."""
    c = DecodeConfig(batch_capacity=6, max_splits=8, max_context=3000, query_heads=hq, kv_heads=8, page_size=page,
                     workers=96)
    lengths = [3000, 1, page, page + 1, 777, 0]
    inputs = W.make_inputs(c, lengths, seed=page)
    expected = OA.paged_attention(*inputs[:3], inputs[3], lengths, c.page_size)
    for kernel in (["valu"] if hq == 32 else []) + ["mfma", "generic"]:
        for mode in (Mode.D1, Mode.R1):
            engine = DecodeEngine(c, force_mode=mode, kernel=kernel)
            out = run(engine, lengths, inputs)
            assert engine.last_kernel == kernel
            close(out[:6], expected[:6], msg=f"page {page} kernel {kernel} mode {mode.name}")
