"""SGLang v0.4.6.post5 attention-backend adapter.  Prefill stays upstream.

Drop-in for src/sglang_decode/integrations/sglang_backend.py:14-108: a subclass of
SGLang's ``TritonAttnBackend`` that routes eligible full-GQA decode steps through
``DecodeEngine`` on the CSR token-index entry (kv_indptr / kv_indices, page_size
1) and keeps the upstream kernel for everything else.  Selected by swapping one
import in SGLang's model_runner.py (``ScheduledTritonBackend as
TritonAttnBackend``).

SGLang is not a dependency: when it is not importable, ``ScheduledTritonBackend``
is None and ``make_backend_class(base)`` builds the same subclass over any base
class that provides the upstream attributes (used by the host-side tests).

Environment: DECODE_DISABLE=1 keeps upstream decode; DECODE_MODE=AUTO|R0|R1|
STATIC|D1|D4 forces a schedule; DECODE_POLICY=<validated policy json> picks the
schedule per batch shape (unset: the artifact shipped for the GPU's architecture,
policies/mi355x.json on gfx950; "none": no rules, R1 as in the reference);
DECODE_BATCH_CAPACITY (default 64); DECODE_REUSE_PLAN=0 rebuilds the plan on
every layer; DECODE_WORKERS overrides the persistent worker count (default: two
per compute unit); DECODE_FUSED_KV=0 keeps upstream's set_kv_buffer and a separate
q copy instead of the one-launch KV write + q staging (kernels/kv_store.py);
DECODE_FUSED_META=0 keeps the reference's per-step copies of kv_indptr differences
and num_kv_splits into the plan (and the active fill) instead of the plan launch
reading them itself (sgd_build_plan_csr).
"""
import os

import torch

from ..config import WORKGROUPS_PER_CU, DecodeConfig, Mode
from ..kernels.kv_store import store_kv_and_stage_q
from ..planning.policy import policy_from_env

try:  # pragma: no cover - depends on an optional install
    from sglang.srt.layers.attention.triton_backend import TritonAttnBackend as _UpstreamBackend
except Exception:  # ImportError, or an sglang import that fails without its own deps
    _UpstreamBackend = None


def eligible_model(model_runner, num_head, num_kv_head):
    """Model-level gates of sglang_backend.py:21-37; returns the KV dtype/head_dim or None."""
    if os.getenv("DECODE_DISABLE", "0") == "1":
        return None
    if getattr(model_runner.server_args, "pp_size", 1) != 1:
        return None
    c = model_runner.model_config
    if (getattr(c, "is_multimodal", False) or getattr(c, "is_encoder_decoder", False)
            or getattr(c, "is_deepseek_mla", False)
            or getattr(model_runner.server_args, "speculative_algorithm", None) is not None):
        return None
    key = model_runner.token_to_kv_pool.get_key_buffer(0)
    value = model_runner.token_to_kv_pool.get_value_buffer(0)
    if key.shape != value.shape or key.dtype not in (torch.float16, torch.bfloat16):
        return None
    if num_head % num_kv_head or num_head // num_kv_head not in (1, 2, 4, 8, 16):
        return None
    if key.shape[-1] not in (64, 128, 256):
        return None
    return key.dtype, key.shape[-1]


def layer_eligible(layer, config):
    """Per-layer gates of sglang_backend.py:84-90."""
    return not (layer.logit_cap > 0 or layer.tp_q_head_num != config.query_heads
                or layer.tp_k_head_num != config.kv_heads or layer.qk_head_dim != config.head_dim
                or layer.v_head_dim != config.head_dim
                or getattr(layer, "sliding_window_size", -1) not in (None, -1))


def _fused_device(t):
    """The fused launches (KV write + q staging, the plan reading the CSR metadata) run on
    the GPU library only."""
    return t.device.type == "cuda"


def make_backend_class(base):
    from ..runtime.engine import DecodeEngine

    class ScheduledTritonBackend(base):
        def __init__(self, model_runner, **kwargs):
            super().__init__(model_runner, **kwargs)
            self.scheduled = None
            self._prepared = False
            self._eligible_step = False
            self.reuse_plan = os.getenv("DECODE_REUSE_PLAN", "1") == "1"
            self.fused_kv = os.getenv("DECODE_FUSED_KV", "1") == "1"
            self.fused_meta = os.getenv("DECODE_FUSED_META", "1") == "1"
            found = eligible_model(model_runner, self.num_head, self.num_kv_head)
            if found is None:
                return
            dtype, head_dim = found
            workers = (int(os.getenv("DECODE_WORKERS", "0"))
                       or WORKGROUPS_PER_CU * max(1, self.device_core_count))
            config = DecodeConfig(
                batch_capacity=int(os.getenv("DECODE_BATCH_CAPACITY", "64")),
                max_splits=self.max_kv_splits, max_context=self.max_context_len,
                query_heads=self.num_head, kv_heads=self.num_kv_head, head_dim=head_dim,
                page_size=1, workers=workers)
            mode_name = os.getenv("DECODE_MODE", "AUTO")
            force = -1 if mode_name == "AUTO" else int(Mode[mode_name])
            rules = policy_from_env(self.device)
            # Indexed by absolute layer_id.
            layers = model_runner.model_config.hf_config.num_hidden_layers
            self.scheduled = DecodeEngine(config, self.device, dtype, layers, rules, force)
            self.query_buffers = [torch.empty_like(x.output) for x in self.scheduled.layers]

        def _begin_step(self, bs, decode, spec_info):
            self._prepared = False
            self._eligible_step = (self.scheduled is not None and decode and spec_info is None
                                   and 0 < bs <= self.scheduled.config.batch_capacity)
            # with the fused metadata read the plan launch sets active itself
            if self._eligible_step and not (self.fused_meta and _fused_device(self.scheduled.plan.active)):
                self.scheduled.plan.active.fill_(bs)

        def init_forward_metadata(self, forward_batch):
            super().init_forward_metadata(forward_batch)
            self._begin_step(forward_batch.batch_size,
                             forward_batch.forward_mode.is_decode_or_idle(), forward_batch.spec_info)

        def init_forward_metadata_capture_cuda_graph(self, bs, num_tokens, req_pool_indices,
                                                     seq_lens, encoder_lens, forward_mode,
                                                     spec_info):
            super().init_forward_metadata_capture_cuda_graph(
                bs, num_tokens, req_pool_indices, seq_lens, encoder_lens, forward_mode, spec_info)
            self._begin_step(bs, forward_mode.is_decode_or_idle(), spec_info)

        def init_forward_metadata_replay_cuda_graph(self, bs, req_pool_indices, seq_lens,
                                                    seq_lens_sum, encoder_lens, forward_mode,
                                                    spec_info, seq_lens_cpu):
            super().init_forward_metadata_replay_cuda_graph(
                bs, req_pool_indices, seq_lens, seq_lens_sum, encoder_lens, forward_mode,
                spec_info, seq_lens_cpu)
            # The host gate picks a captured bucket; captured nodes rebuild the device plan.
            self._begin_step(bs, forward_mode.is_decode_or_idle(), spec_info)

        def forward_decode(self, q, k, v, layer, forward_batch, save_kv_cache=True):
            # Graph runners may warm up repeatedly after one metadata hook: re-arm on
            # layer 0 so every capture records the plan build.
            if layer.layer_id == 0:
                self._prepared = False
            engine = self.scheduled
            if not self._eligible_step or not layer_eligible(layer, engine.config):
                return super().forward_decode(q, k, v, layer, forward_batch, save_kv_cache)
            pool, c = forward_batch.token_to_kv_pool, engine.config
            kbuf, vbuf = pool.get_key_buffer(layer.layer_id), pool.get_value_buffer(layer.layer_id)
            batch = q.shape[0]
            fused = self.fused_kv and _fused_device(q)
            k_new = v_new = None
            if save_kv_cache:
                if fused and k.dtype == kbuf.dtype and v.dtype == vbuf.dtype:
                    # written by the launch below, together with the q staging (a pool
                    # whose storage type differs from k's keeps upstream's conversion)
                    k_new = k.view(batch, c.kv_heads, c.head_dim)
                    v_new = v.view(batch, c.kv_heads, c.head_dim)
                else:
                    pool.set_kv_buffer(layer, forward_batch.out_cache_loc, k, v)
            meta, p = self.forward_metadata, engine.plan
            if not self._prepared or not self.reuse_plan:
                if self.fused_meta and _fused_device(p.active):
                    # lengths = kv_indptr differences, splits and active read inside the plan launch
                    engine.prepare(csr_metadata=(meta.kv_indptr, meta.num_kv_splits, batch))
                else:
                    p.lengths[:batch].copy_(meta.kv_indptr[1:batch + 1] - meta.kv_indptr[:batch])
                    p.splits[:batch].copy_(meta.num_kv_splits[:batch])
                    engine.prepare()
                self._prepared = True
            qbuf = self.query_buffers[layer.layer_id]
            q_view = q.view(batch, c.query_heads, c.head_dim)
            if fused:
                store_kv_and_stage_q(k_new, v_new, forward_batch.out_cache_loc, kbuf, vbuf, q_view, qbuf)
            else:
                qbuf[:batch].copy_(q_view)
            out = engine.execute(qbuf, kbuf, vbuf, meta.kv_indices, layer=layer.layer_id, indptr=meta.kv_indptr,
                                 scale=layer.scaling)
            return out[:batch].view(batch, -1)

    return ScheduledTritonBackend


ScheduledTritonBackend = make_backend_class(_UpstreamBackend) if _UpstreamBackend is not None else None
