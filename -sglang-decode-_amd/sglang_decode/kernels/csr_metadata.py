"""The step's CSR metadata (kv_indptr, kv_indices, num_kv_splits) from the request pool in
one launch (kernel in csrc/csr_metadata.hip), optionally also the plan's inputs.

What the reference adapter consumes (integrations/sglang_backend.py:98-107) and upstream
SGLang's triton backend produces before it: kv_indptr[1:] = cumsum(seq_lens), kv_indices =
the rows req_to_token[req_pool_indices[i], :seq_lens[i]] back to back, and split counts --
here by the reference harness rule (benchmarks/workloads.py:20-21).
"""
import ctypes

import torch

from .. import _lib
from .._lib import check, ptr


def csr_metadata(seq_lens, req_pool_indices, req_to_token, max_splits, kv_indptr, kv_indices,
                 num_kv_splits=None, plan=None, error=None):
    """Writes kv_indptr [>= batch + 1] and kv_indices (its length is the capacity), and
    num_kv_splits [>= batch] when given; with ``plan`` (PlanBuffers) also plan.lengths /
    plan.splits rows < batch and plan.active.  ``error``: optional int32 [1], set to 1 for
    an invalid row or a total beyond the capacity (never cleared here).  Host misuse raises
    ValueError before any launch."""
    batch = seq_lens.shape[0]
    dev = kv_indptr.device
    if seq_lens.dim() != 1 or req_pool_indices.shape != seq_lens.shape:
        raise ValueError("csr_metadata: seq_lens and req_pool_indices must be [batch]")
    for name, t in (("seq_lens", seq_lens), ("req_pool_indices", req_pool_indices)):
        if t.dtype not in (torch.int32, torch.int64) or t.device != dev:
            raise ValueError(f"csr_metadata: {name} must be int32/int64 on {dev}")
    if req_to_token.dim() != 2 or req_to_token.dtype != torch.int32 or req_to_token.stride(1) != 1 \
            or req_to_token.device != dev:
        raise ValueError("csr_metadata: req_to_token must be int32 [rows, cols] with unit column stride")
    outs = [("kv_indptr", kv_indptr, batch + 1), ("kv_indices", kv_indices, 0)]
    if num_kv_splits is not None:
        outs.append(("num_kv_splits", num_kv_splits, batch))
    if error is not None:
        outs.append(("error", error, 1))
    for name, t, need in outs:
        if t.dtype != torch.int32 or t.dim() != 1 or not t.is_contiguous() or t.shape[0] < need or t.device != dev:
            raise ValueError(f"csr_metadata: {name} must be contiguous int32 [>= {need}] on {dev}")
    pl = ps = pa = None
    if plan is not None:
        if plan.device != dev or batch > plan.config.batch_capacity:
            raise ValueError("csr_metadata: the plan must be on the same device and hold the batch")
        pl, ps, pa = plan.lengths, plan.splits, plan.active
    seq_lens, req_pool_indices = seq_lens.contiguous(), req_pool_indices.contiguous()
    check(_lib.lib().sgd_csr_metadata(
        ptr(seq_lens), int(seq_lens.dtype == torch.int64), ptr(req_pool_indices),
        int(req_pool_indices.dtype == torch.int64), ptr(req_to_token), req_to_token.shape[0],
        req_to_token.stride(0), req_to_token.shape[1], batch, int(max_splits), ptr(kv_indptr), ptr(kv_indices),
        kv_indices.shape[0], ptr(num_kv_splits), ptr(pl), ptr(ps), ptr(pa), ptr(error),
        _lib.stream_handle(dev)), "csr_metadata")
