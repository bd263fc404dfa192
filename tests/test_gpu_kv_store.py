"""The one-launch KV-pool write + q staging (csrc/kv_store.hip) against torch's scatter and
copy -- what the reference adapter runs (integrations/sglang_backend.py:91-92, 102-103):
bit-exact, for int32 and int64 slots, strided sources (q/k/v as views of one packed
projection output), q-only and KV-only launches, slots outside the pool, and the
adapter end to end with the new tokens written and attended in the same step."""
import types

import pytest
import torch

from sglang_decode.kernels.kv_store import store_kv_and_stage_q

pytestmark = pytest.mark.gpu

DEV = "cuda"


def pools(tokens, hkv, d, dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    k = torch.randn((tokens, hkv, d), generator=g, device=DEV, dtype=torch.float32).to(dtype)
    v = torch.randn((tokens, hkv, d), generator=g, device=DEV, dtype=torch.float32).to(dtype)
    return k, v


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("loc_dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (64, 8, 128), (8, 8, 64), (16, 4, 256)])
def test_store_and_stage_match_torch(dtype, loc_dtype, hq, hkv, d):
    batch, tokens = 37, 5000
    kc, vc = pools(tokens, hkv, d, dtype, 1)
    g = torch.Generator(device=DEV).manual_seed(2)
    # one packed projection output [batch, (hq + 2 hkv) * d]: q, k, v are strided views
    qkv = torch.randn((batch, (hq + 2 * hkv) * d), generator=g, device=DEV, dtype=torch.float32).to(dtype)
    q = qkv[:, :hq * d].view(batch, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].view(batch, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(batch, hkv, d)
    loc = torch.randperm(tokens, generator=torch.Generator().manual_seed(3))[:batch].to(loc_dtype).to(DEV)
    qbuf = torch.full((64, hq, d), 7.0, device=DEV, dtype=dtype)
    ek, ev, eq = kc.clone(), vc.clone(), qbuf.clone()
    ek[loc.long()] = k
    ev[loc.long()] = v
    eq[:batch].copy_(q)
    store_kv_and_stage_q(k, v, loc, kc, vc, q, qbuf)
    torch.cuda.synchronize()
    assert torch.equal(kc, ek) and torch.equal(vc, ev) and torch.equal(qbuf, eq)


def test_parts_and_out_of_range_slots():
    batch, tokens, hq, hkv, d = 6, 300, 32, 8, 128
    kc, vc = pools(tokens, hkv, d, torch.bfloat16, 4)
    before_k, before_v = kc.clone(), vc.clone()
    k = torch.randn((batch, hkv, d), device=DEV).to(torch.bfloat16)
    v = torch.randn((batch, hkv, d), device=DEV).to(torch.bfloat16)
    q = torch.randn((batch, hq, d), device=DEV).to(torch.bfloat16)
    qbuf = torch.zeros((8, hq, d), device=DEV, dtype=torch.bfloat16)
    # q only: the pools are untouched
    store_kv_and_stage_q(q_in=q, q_out=qbuf)
    torch.cuda.synchronize()
    assert torch.equal(qbuf[:batch], q) and not qbuf[batch:].any()
    assert torch.equal(kc, before_k) and torch.equal(vc, before_v)
    # KV only, with two slots outside [0, tokens): those rows are skipped
    loc = torch.tensor([5, -1, 299, tokens, 0, 17], dtype=torch.int64, device=DEV)
    store_kv_and_stage_q(k, v, loc, kc, vc)
    torch.cuda.synchronize()
    ek, ev = before_k.clone(), before_v.clone()
    for b, slot in enumerate(loc.tolist()):
        if 0 <= slot < tokens:
            ek[slot], ev[slot] = k[b], v[b]
    assert torch.equal(kc, ek) and torch.equal(vc, ev)
    # host-checkable misuse raises before any launch
    with pytest.raises(ValueError):
        store_kv_and_stage_q(k, v, loc, kc, vc.float())
    with pytest.raises(ValueError):
        store_kv_and_stage_q(k, v, None, kc, vc)
    with pytest.raises(ValueError):
        store_kv_and_stage_q(q_in=q, q_out=qbuf[:2])


def test_adapter_writes_new_tokens_and_attends_them():
    """The adapter's decode with save_kv_cache: each request's newest token goes to its
    slot in this step's launch and is part of this step's attention (oracle on the
    pools after the write)."""
    from oracle import attention as OA
    from sglang_decode import workloads as W
    from gpu_util import close
    from test_sglang_adapter import Backend, FakeMode, layer, model_runner
    mr = model_runner(device=DEV, tokens=4096)
    gen = torch.Generator(device=DEV).manual_seed(7)
    for t in mr.token_to_kv_pool.keys + mr.token_to_kv_pool.values:
        t.copy_(torch.randn(t.shape, generator=gen, device=DEV, dtype=torch.float32))
    mr.token_to_kv_pool.set_kv_buffer = None  # the fused launch must do the write
    b = Backend(mr)
    lengths = [700, 33, 1, 2048]
    splits = W.split_hints(lengths, 8)
    perm = torch.randperm(4096, generator=torch.Generator().manual_seed(5))[:sum(lengths)].to(torch.int32)
    indptr = torch.zeros(len(lengths) + 1, dtype=torch.int32)
    indptr[1:] = torch.cumsum(torch.tensor(lengths), 0)
    newest = perm[indptr[1:].long() - 1].to(torch.int64).cuda()  # each request's last slot
    b.forward_metadata = types.SimpleNamespace(kv_indptr=indptr.cuda(), kv_indices=perm.cuda(),
                                               num_kv_splits=torch.tensor(splits, dtype=torch.int32).cuda())
    fb = types.SimpleNamespace(batch_size=4, forward_mode=FakeMode(True), spec_info=None, out_cache_loc=newest,
                               token_to_kv_pool=mr.token_to_kv_pool)
    b.init_forward_metadata(fb)
    for lid in range(2):
        q = torch.randn(4, 32 * 128, generator=gen, device=DEV, dtype=torch.float32).to(torch.bfloat16)
        k = torch.randn(4, 8 * 128, generator=gen, device=DEV, dtype=torch.float32).to(torch.bfloat16)
        v = torch.randn(4, 8 * 128, generator=gen, device=DEV, dtype=torch.float32).to(torch.bfloat16)
        out = b.forward_decode(q, k, v, layer(lid), fb, save_kv_cache=True)
        torch.cuda.synchronize()
        keys, values = mr.token_to_kv_pool.keys[lid], mr.token_to_kv_pool.values[lid]
        assert torch.equal(keys[newest], k.view(4, 8, 128)) and torch.equal(values[newest], v.view(4, 8, 128))
        exp = OA.csr_attention(q.view(4, 32, 128), keys, values, indptr, perm, lengths, scale=0.125)
        close(out.view(4, 32, 128), exp[:4])


def test_adapter_decode_under_graph_replay():
    """SGLang's graph runner: the metadata hook, then every layer's forward_decode captured
    once at a batch bucket and replayed after new contents of the runner's fixed buffers
    (kv_indptr, kv_indices, num_kv_splits, out_cache_loc, q/k/v).  Each replay writes the
    new tokens into the pools and attends them, with the plan read from the metadata inside
    the captured plan launch (oracle on the pools after the write)."""
    from oracle import attention as OA
    from sglang_decode import workloads as W
    from gpu_util import close
    from test_sglang_adapter import Backend, FakeMode, layer, model_runner
    bs, tokens, layers = 4, 4096, 2
    mr = model_runner(device=DEV, tokens=tokens, layers=layers)
    gen = torch.Generator(device=DEV).manual_seed(11)
    pool = mr.token_to_kv_pool
    for t in pool.keys + pool.values:
        t.copy_(torch.randn(t.shape, generator=gen, device=DEV, dtype=torch.float32))
    pool.set_kv_buffer = None  # the fused launch must do the write
    b = Backend(mr)
    indptr = torch.zeros(bs + 1, dtype=torch.int32, device=DEV)
    indices = torch.zeros(tokens, dtype=torch.int32, device=DEV)
    splits = torch.ones(bs, dtype=torch.int32, device=DEV)
    loc = torch.zeros(bs, dtype=torch.int64, device=DEV)
    q = torch.zeros(bs, 32 * 128, dtype=torch.bfloat16, device=DEV)
    kv = [(torch.zeros(bs, 8 * 128, dtype=torch.bfloat16, device=DEV),
           torch.zeros(bs, 8 * 128, dtype=torch.bfloat16, device=DEV)) for _ in range(layers)]
    b.forward_metadata = types.SimpleNamespace(kv_indptr=indptr, kv_indices=indices, num_kv_splits=splits)
    fb = types.SimpleNamespace(batch_size=bs, forward_mode=FakeMode(True), spec_info=None, out_cache_loc=loc,
                               token_to_kv_pool=pool)

    def set_step(lengths, seed):
        perm = torch.randperm(tokens, generator=torch.Generator().manual_seed(seed))[:sum(lengths)].to(torch.int32)
        ip = torch.zeros(bs + 1, dtype=torch.int32)
        ip[1:] = torch.cumsum(torch.tensor(lengths), 0)
        indptr.copy_(ip)
        indices[:perm.numel()].copy_(perm)
        splits.copy_(torch.tensor(W.split_hints(lengths, 8), dtype=torch.int32))
        loc.copy_(perm[ip[1:].long() - 1].to(torch.int64))  # each request's newest token
        for x in [q] + [t for pair in kv for t in pair]:
            x.copy_(torch.randn(x.shape, generator=gen, device=DEV, dtype=torch.float32))
        return ip, perm

    def run():
        return [b.forward_decode(q, kv[lid][0], kv[lid][1], layer(lid), fb, save_kv_cache=True)
                for lid in range(layers)]

    steps = [[700, 33, 1, 2048], [1, 1, 1, 1], [1024, 1024, 1000, 1000], [5, 4000, 17, 64]]
    set_step(steps[0], 0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        b.init_forward_metadata_capture_cuda_graph(bs, bs, None, None, None, FakeMode(True), None)
        run()  # eager warm-up outside the capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            outs = run()
    torch.cuda.synchronize()
    for i, lengths in enumerate(steps):
        ip, perm = set_step(lengths, i + 1)
        b.init_forward_metadata_replay_cuda_graph(bs, None, None, 0, None, FakeMode(True), None, None)
        g.replay()
        torch.cuda.synchronize()
        newest = loc.long()
        for lid in range(layers):
            keys, values = pool.keys[lid], pool.values[lid]
            assert torch.equal(keys[newest], kv[lid][0].view(bs, 8, 128))
            assert torch.equal(values[newest], kv[lid][1].view(bs, 8, 128))
            exp = OA.csr_attention(q.view(bs, 32, 128), keys, values, ip, perm, lengths, scale=0.125)
            close(outs[lid].view(bs, 32, 128), exp[:bs], msg=f"step {i} layer {lid}")
