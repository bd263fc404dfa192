"""SGLang adapter (integrations/sglang_backend.py of the reference, :14-108) over a
stand-in upstream backend: SGLang v0.4.6.post5 is not installed here, so the base class
is a small fake exposing the attributes and hooks the adapter uses.

Host tests check the model / layer / step gates, the environment switches, plan reuse
across layers and what each hook hands the engine; the GPU test runs the adapter end to
end on the CSR entry against the FP32 oracle.  Parity with real SGLang is unpinned."""
import types

import pytest
import torch

from sglang_decode.config import Mode
from sglang_decode.integrations.sglang_backend import make_backend_class


class FakeMode:
    def __init__(self, decode):
        self.decode = decode

    def is_decode_or_idle(self):
        return self.decode


class FakePool:
    def __init__(self, keys, values):
        self.keys, self.values, self.writes = keys, values, []

    def get_key_buffer(self, layer_id):
        return self.keys[layer_id]

    def get_value_buffer(self, layer_id):
        return self.values[layer_id]

    def set_kv_buffer(self, layer, loc, k, v):
        self.writes.append(layer.layer_id)


class FakeUpstream:
    """The TritonAttnBackend surface the adapter relies on."""

    def __init__(self, model_runner, **kwargs):
        self.num_head = model_runner.num_head
        self.num_kv_head = model_runner.num_kv_head
        self.max_kv_splits = 8
        self.max_context_len = 4096
        self.device = model_runner.device
        self.device_core_count = 4
        self.forward_metadata = None
        self.calls = []

    def init_forward_metadata(self, forward_batch):
        self.calls.append("init")

    def init_forward_metadata_capture_cuda_graph(self, *args):
        self.calls.append("capture")

    def init_forward_metadata_replay_cuda_graph(self, *args):
        self.calls.append("replay")

    def forward_decode(self, q, k, v, layer, forward_batch, save_kv_cache=True):
        self.calls.append(("upstream", layer.layer_id))
        return "upstream"


Backend = make_backend_class(FakeUpstream)


def model_runner(device="cpu", heads=32, kv_heads=8, head_dim=128, dtype=torch.bfloat16, layers=2,
                 tokens=64, **flags):
    shape = (tokens, kv_heads, head_dim)
    keys = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(layers)]
    values = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(layers)]
    cfg = types.SimpleNamespace(is_multimodal=flags.get("multimodal", False),
                                is_encoder_decoder=False, is_deepseek_mla=flags.get("mla", False),
                                hf_config=types.SimpleNamespace(num_hidden_layers=layers))
    args = types.SimpleNamespace(pp_size=flags.get("pp", 1), speculative_algorithm=flags.get("spec"))
    return types.SimpleNamespace(num_head=heads, num_kv_head=kv_heads, device=device, model_config=cfg,
                                 server_args=args, token_to_kv_pool=FakePool(keys, values))


def layer(layer_id, heads=32, kv_heads=8, head_dim=128, **kw):
    return types.SimpleNamespace(layer_id=layer_id, logit_cap=kw.get("logit_cap", 0.0),
                                 tp_q_head_num=heads, tp_k_head_num=kv_heads, qk_head_dim=head_dim,
                                 v_head_dim=head_dim, sliding_window_size=kw.get("window", -1),
                                 scaling=0.125)


@pytest.fixture(autouse=True)
def clean_env(monkeypatch):
    for name in ("DECODE_DISABLE", "DECODE_MODE", "DECODE_POLICY", "DECODE_BATCH_CAPACITY",
                 "DECODE_REUSE_PLAN", "DECODE_WORKERS", "DECODE_FUSED_KV", "DECODE_FUSED_META"):
        monkeypatch.delenv(name, raising=False)


def test_eligible_model_builds_engine_from_upstream_geometry(monkeypatch):
    monkeypatch.setenv("DECODE_BATCH_CAPACITY", "16")
    monkeypatch.setenv("DECODE_WORKERS", "24")
    monkeypatch.setenv("DECODE_MODE", "D4")
    b = Backend(model_runner())
    c = b.scheduled.config
    assert (c.batch_capacity, c.max_splits, c.max_context, c.query_heads, c.kv_heads, c.head_dim,
            c.page_size, c.workers) == (16, 8, 4096, 32, 8, 128, 1, 24)
    assert b.scheduled.force_mode == int(Mode.D4)
    assert len(b.scheduled.layers) == 2 and len(b.query_buffers) == 2
    # default workers: two per compute unit
    monkeypatch.delenv("DECODE_WORKERS")
    assert Backend(model_runner()).scheduled.config.workers == 2 * 4


@pytest.mark.parametrize("flags", [dict(mla=True), dict(multimodal=True), dict(spec="eagle"), dict(pp=2),
                                   dict(heads=24, kv_heads=8), dict(head_dim=96), dict(dtype=torch.float32)])
def test_ineligible_models_keep_upstream(flags):
    b = Backend(model_runner(**flags))
    assert b.scheduled is None
    fb = types.SimpleNamespace(batch_size=2, forward_mode=FakeMode(True), spec_info=None)
    b.init_forward_metadata(fb)
    assert b.forward_decode(None, None, None, layer(0), fb) == "upstream"


def test_disable_switch(monkeypatch):
    monkeypatch.setenv("DECODE_DISABLE", "1")
    assert Backend(model_runner()).scheduled is None


class Recorder:
    """Stands in for the engine's device work on a CPU-only host."""

    def __init__(self, engine):
        self.prepares, self.executes, self.metadata = 0, [], []
        engine.prepare = self.prepare
        engine.execute = self.execute
        self.engine = engine

    def prepare(self, *, csr_metadata=None):
        self.prepares += 1
        self.metadata.append(csr_metadata)

    def execute(self, q, k, v, pages, layer=0, *, indptr=None, scale=None):
        self.executes.append(dict(q=q.clone(), k=k, v=v, pages=pages, layer=layer, indptr=indptr,
                                  scale=scale))
        return self.engine.layers[layer].output


def decode_batch(b, lengths, splits):
    indptr = torch.zeros(len(lengths) + 1, dtype=torch.int32)
    indptr[1:] = torch.cumsum(torch.tensor(lengths), 0)
    b.forward_metadata = types.SimpleNamespace(kv_indptr=indptr, kv_indices=torch.arange(sum(lengths),
                                                                                         dtype=torch.int32),
                                               num_kv_splits=torch.tensor(splits, dtype=torch.int32))
    return types.SimpleNamespace(batch_size=len(lengths), forward_mode=FakeMode(True), spec_info=None,
                                 out_cache_loc=None, token_to_kv_pool=b.mr_pool)


def make_backend(**kw):
    mr = model_runner(**kw)
    b = Backend(mr)
    b.mr_pool = mr.token_to_kv_pool
    return b


@pytest.mark.parametrize("reuse", ["1", "0"])
def test_decode_step_data_flow_and_plan_reuse(monkeypatch, reuse):
    monkeypatch.setenv("DECODE_REUSE_PLAN", reuse)
    b = make_backend()
    rec = Recorder(b.scheduled)
    fb = decode_batch(b, [5, 17, 3], [1, 2, 1])
    b.init_forward_metadata(fb)
    assert b.scheduled.plan.active.item() == 3
    q = torch.randn(3, 32 * 128).to(torch.bfloat16)
    for lid in range(2):
        out = b.forward_decode(q, q, q, layer(lid), fb, save_kv_cache=True)
        assert out.shape == (3, 32 * 128)
    p = b.scheduled.plan
    assert p.lengths[:3].tolist() == [5, 17, 3] and p.splits[:3].tolist() == [1, 2, 1]
    assert rec.prepares == (1 if reuse == "1" else 2)  # one plan per step unless reuse is off
    assert [e["layer"] for e in rec.executes] == [0, 1]
    e = rec.executes[1]
    assert e["indptr"] is b.forward_metadata.kv_indptr and e["pages"] is b.forward_metadata.kv_indices
    assert e["k"] is b.mr_pool.keys[1] and e["scale"] == 0.125
    assert torch.equal(e["q"][:3], q.view(3, 32, 128))  # per-layer q buffer at capture capacity
    assert e["q"].shape == (64, 32, 128)
    assert b.mr_pool.writes == [0, 1]


def test_fused_metadata_read_replaces_the_plan_copies(monkeypatch):
    """With the plan launch reading kv_indptr / num_kv_splits itself (the default on the
    GPU), the adapter makes no copies into the plan and no active fill; the plan build
    gets the step's metadata and batch.  DECODE_FUSED_META=0 restores the copies."""
    from sglang_decode.integrations import sglang_backend as SB
    monkeypatch.setattr(SB, "_fused_device", lambda t: True)
    monkeypatch.setenv("DECODE_FUSED_KV", "0")
    b = make_backend()
    rec = Recorder(b.scheduled)
    p = b.scheduled.plan
    p.lengths.fill_(-7)
    p.active.fill_(-7)
    fb = decode_batch(b, [5, 17, 3], [1, 2, 1])
    b.init_forward_metadata(fb)
    assert p.active.item() == -7  # left to the plan launch
    q = torch.randn(3, 32 * 128).to(torch.bfloat16)
    for lid in range(2):
        b.forward_decode(q, q, q, layer(lid), fb, save_kv_cache=False)
    assert rec.prepares == 1 and (p.lengths == -7).all()
    indptr, splits, batch = rec.metadata[0]
    assert indptr is b.forward_metadata.kv_indptr and splits is b.forward_metadata.num_kv_splits and batch == 3
    monkeypatch.setenv("DECODE_FUSED_META", "0")
    b = make_backend()
    rec = Recorder(b.scheduled)
    fb = decode_batch(b, [5, 17, 3], [1, 2, 1])
    b.init_forward_metadata(fb)
    b.forward_decode(q, q, q, layer(0), fb, save_kv_cache=False)
    p = b.scheduled.plan
    assert rec.metadata == [None] and p.active.item() == 3
    assert p.lengths[:3].tolist() == [5, 17, 3] and p.splits[:3].tolist() == [1, 2, 1]


class StoreRecorder:
    """Stands in for the one-launch KV write + q staging on a CPU-only host."""

    def __init__(self):
        self.calls = []

    def __call__(self, k_new, v_new, loc, k_cache, v_cache, q_in, q_out):
        self.calls.append(dict(k_new=k_new, v_new=v_new, loc=loc, k_cache=k_cache, v_cache=v_cache, q_in=q_in,
                               q_out=q_out))
        q_out[:q_in.shape[0]].copy_(q_in)


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float32])
def test_fused_kv_write_and_q_staging(monkeypatch, kv_dtype):
    """On the GPU the adapter replaces set_kv_buffer and the q copy with one launch
    (kernels/kv_store.py); a k/v dtype other than the pool's keeps set_kv_buffer (its
    conversion) while q is still staged by the launch."""
    from sglang_decode.integrations import sglang_backend as SB
    store = StoreRecorder()
    monkeypatch.setattr(SB, "store_kv_and_stage_q", store)
    monkeypatch.setattr(SB, "_fused_device", lambda t: True)
    b = make_backend()
    rec = Recorder(b.scheduled)
    fb = decode_batch(b, [5, 17, 3], [1, 2, 1])
    fb.out_cache_loc = torch.tensor([4, 21, 24], dtype=torch.int64)
    b.init_forward_metadata(fb)
    q = torch.randn(3, 32 * 128).to(torch.bfloat16)
    kv = torch.randn(3, 8 * 128).to(kv_dtype)
    for lid in range(2):
        b.forward_decode(q, kv, kv, layer(lid), fb, save_kv_cache=True)
    assert [e["layer"] for e in rec.executes] == [0, 1]
    assert len(store.calls) == 2
    for lid, call in enumerate(store.calls):
        assert call["q_out"] is b.query_buffers[lid] and call["k_cache"] is b.mr_pool.keys[lid]
        assert call["v_cache"] is b.mr_pool.values[lid] and call["loc"] is fb.out_cache_loc
        assert torch.equal(call["q_in"], q.view(3, 32, 128))
        assert rec.executes[lid]["k"] is b.mr_pool.keys[lid]
        if kv_dtype == torch.bfloat16:
            assert call["k_new"].shape == (3, 8, 128) and torch.equal(call["k_new"], kv.view(3, 8, 128))
        else:
            assert call["k_new"] is None and call["v_new"] is None
    assert b.mr_pool.writes == ([] if kv_dtype == torch.bfloat16 else [0, 1])
    # DECODE_FUSED_KV=0: upstream set_kv_buffer and a separate q copy
    monkeypatch.setenv("DECODE_FUSED_KV", "0")
    b = make_backend()
    Recorder(b.scheduled)
    fb = decode_batch(b, [5, 17, 3], [1, 2, 1])
    b.init_forward_metadata(fb)
    store.calls.clear()
    b.forward_decode(q, kv, kv, layer(0), fb, save_kv_cache=True)
    assert store.calls == [] and b.mr_pool.writes == [0]


def test_step_and_layer_gates_fall_back_to_upstream():
    b = make_backend()
    Recorder(b.scheduled)
    q = torch.zeros(2, 32 * 128, dtype=torch.bfloat16)
    # prefill / extend step
    fb = decode_batch(b, [4, 4], [1, 1])
    fb.forward_mode = FakeMode(False)
    b.init_forward_metadata(fb)
    assert b.forward_decode(q, q, q, layer(0), fb) == "upstream"
    # speculative step, and a batch beyond the capture capacity
    for change in (dict(spec_info=object()), dict(batch_size=65)):
        fb = decode_batch(b, [4, 4], [1, 1])
        for k, v in change.items():
            setattr(fb, k, v)
        b.init_forward_metadata(fb)
        assert b.forward_decode(q, q, q, layer(0), fb) == "upstream"
    # per-layer gates on an eligible step
    fb = decode_batch(b, [4, 4], [1, 1])
    b.init_forward_metadata(fb)
    for bad in (layer(0, logit_cap=30.0), layer(0, window=4096), layer(0, heads=16), layer(0, head_dim=64)):
        assert b.forward_decode(q, q, q, bad, fb) == "upstream"
    assert not isinstance(b.forward_decode(q, q, q, layer(0), fb), str)


def test_graph_hooks_call_upstream_and_arm_the_step():
    b = make_backend()
    b.init_forward_metadata_capture_cuda_graph(8, 8, None, None, None, FakeMode(True), None)
    assert b._eligible_step and b.scheduled.plan.active.item() == 8
    b.init_forward_metadata_replay_cuda_graph(3, None, None, 0, None, FakeMode(True), None, None)
    assert b._eligible_step and b.scheduled.plan.active.item() == 3
    b.init_forward_metadata_replay_cuda_graph(100, None, None, 0, None, FakeMode(True), None, None)
    assert not b._eligible_step
    assert b.calls == ["capture", "replay", "replay"]


@pytest.mark.gpu
def test_adapter_end_to_end_on_gpu():
    from oracle import attention as OA
    from sglang_decode import workloads as W
    from gpu_util import close
    mr = model_runner(device="cuda", tokens=4096)
    gen = torch.Generator(device="cuda").manual_seed(3)
    for t in mr.token_to_kv_pool.keys + mr.token_to_kv_pool.values:
        t.copy_(torch.randn(t.shape, generator=gen, device="cuda", dtype=torch.float32))
    b = Backend(mr)
    lengths = [700, 33, 1, 2048]
    splits = W.split_hints(lengths, 8)
    perm = torch.randperm(4096, generator=torch.Generator().manual_seed(5))[:sum(lengths)].to(torch.int32)
    indptr = torch.zeros(len(lengths) + 1, dtype=torch.int32)
    indptr[1:] = torch.cumsum(torch.tensor(lengths), 0)
    b.forward_metadata = types.SimpleNamespace(kv_indptr=indptr.cuda(), kv_indices=perm.cuda(),
                                               num_kv_splits=torch.tensor(splits, dtype=torch.int32).cuda())
    fb = types.SimpleNamespace(batch_size=4, forward_mode=FakeMode(True), spec_info=None, out_cache_loc=None,
                               token_to_kv_pool=mr.token_to_kv_pool)
    b.init_forward_metadata(fb)
    for lid in range(2):
        q = torch.randn(4, 32 * 128, generator=gen, device="cuda", dtype=torch.float32).to(torch.bfloat16)
        out = b.forward_decode(q, None, None, layer(lid), fb, save_kv_cache=False)
        torch.cuda.synchronize()
        exp = OA.csr_attention(q.view(4, 32, 128), mr.token_to_kv_pool.keys[lid],
                               mr.token_to_kv_pool.values[lid], indptr, perm, lengths, scale=0.125)
        close(out.view(4, 32, 128), exp[:4])
