"""Seeded synthetic decode workloads (the five benchmark configurations) and input fixtures.

The split rule is the reference harness's (benchmarks/workloads.py:14-21):
``chunk = ceil(max(L) / maximum)``, ``S_r = clamp(ceil(L_r / chunk), 1, maximum)``.
Input generation differs from benchmarks/workloads.py:24-40 on purpose: lengths
come from numpy's PCG64 and Q/K/V from a seeded torch CPU generator (or, for the
multi-GiB pools, a seeded device generator), so host and device see identical
bytes without a device RNG on the CPU side.

Configurations (batch, q heads / kv heads, head_dim 128):

* ``c1``: batch 4, 8/2, CSR page 1, L ~ U[16, 256], max_context 256.
* ``c2``: batch 64, 32/8, CSR page 1, L = clip(round(exp(N(ln 1024, 0.8))), 128, 8192),
  1M-token pool with randomly permuted slots.
* ``c3``: batch 128, 32/8, two 32768-token requests + 126 x U[32, 512], splits of at most
  512 tokens (``split_hints(L, 64)``), max_splits 64.
* ``c4``: batch 32, 64/8, page_size 16, L ~ U[2048, 16384], page table slices of a random
  permutation of a 200k-page pool.
* ``c5``: 32 layers, 32/8, batch 64 -> 48 -> 17 -> 1, L from lognormal(median 2048) growing by 1
  per step.
"""
import math
import numpy as np

from .config import DecodeConfig

LOGNORMAL_SIGMA = 0.8


def split_hints(lengths, maximum=16):
    chunk = max(1, math.ceil(max(lengths, default=0) / maximum))
    return [max(1, min(maximum, math.ceil(n / chunk))) for n in lengths]


def _rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def c1_lengths(seed=101):
    return [int(x) for x in _rng(seed).integers(16, 257, size=4)]


def lognormal_lengths(batch, median, lo, hi, seed):
    x = np.exp(_rng(seed).normal(math.log(median), LOGNORMAL_SIGMA, size=batch))
    return [int(v) for v in np.clip(np.rint(x), lo, hi)]


def c2_lengths(seed=202):
    return lognormal_lengths(64, 1024, 128, 8192, seed)


def c3_lengths(seed=303):
    return [32768, 32768] + [int(x) for x in _rng(seed).integers(32, 513, size=126)]


def c4_lengths(seed=404):
    return [int(x) for x in _rng(seed).integers(2048, 16385, size=32)]


def c5_lengths(seed=505):
    return lognormal_lengths(64, 2048, 128, 16384, seed)


C5_BATCHES = (64, 48, 17, 1)


def config_for(name, workers=256):
    """DecodeConfig of each benchmark configuration."""
    if name == "c1":
        return DecodeConfig(batch_capacity=4, max_splits=16, max_context=256, query_heads=8,
                            kv_heads=2, head_dim=128, page_size=1, workers=workers)
    if name == "c2":
        return DecodeConfig(batch_capacity=64, max_splits=16, max_context=8192, query_heads=32,
                            kv_heads=8, head_dim=128, page_size=1, workers=workers)
    if name == "c3":
        return DecodeConfig(batch_capacity=128, max_splits=64, max_context=32768,
                            query_heads=32, kv_heads=8, head_dim=128, page_size=1,
                            workers=workers)
    if name == "c4":
        return DecodeConfig(batch_capacity=32, max_splits=16, max_context=16384, query_heads=64,
                            kv_heads=8, head_dim=128, page_size=16, workers=workers)
    if name == "c5":
        return DecodeConfig(batch_capacity=64, max_splits=16, max_context=32768,
                            query_heads=32, kv_heads=8, head_dim=128, page_size=1,
                            workers=workers)
    raise KeyError(name)


def lengths_for(name):
    return {"c1": c1_lengths, "c2": c2_lengths, "c3": c3_lengths, "c4": c4_lengths,
            "c5": c5_lengths}[name]()


def splits_for(name, lengths, config):
    return split_hints(lengths, config.max_splits)


# ---------------------------------------------------------------- tensors (torch)

def _torch():
    import torch
    return torch


def make_inputs(config, lengths, seed=17, device="cuda", dtype=None, pool_pages=None,
                device_pool=False):
    """Paged fixture: (q [Bcap,Hq,D], k/v [pages, page, Hkv, D], table [Bcap, max_pages]).

    Pages are a seeded random permutation of a pool of ``pool_pages`` pages (at least the
    pages the batch needs); unused table entries are -1.  Generated on the CPU, or, with
    ``device_pool``, the (large) K/V pools are drawn by a seeded generator on ``device``.
    """
    torch = _torch()
    dtype = torch.bfloat16 if dtype is None else dtype
    g = torch.Generator().manual_seed(seed)
    per_request = [math.ceil(n / config.page_size) for n in lengths]
    pool = max(1, sum(per_request), pool_pages or 0)
    perm = torch.randperm(pool, generator=g)
    table = torch.full((config.batch_capacity, config.max_pages), -1, dtype=torch.int32)
    cursor = 0
    for row, count in enumerate(per_request):
        table[row, :count] = perm[cursor:cursor + count].to(torch.int32)
        cursor += count
    shape = (pool, config.page_size, config.kv_heads, config.head_dim)
    if device_pool:
        dg = torch.Generator(device=device).manual_seed(seed + 1)
        k = torch.randn(shape, generator=dg, device=device, dtype=dtype)
        v = torch.randn(shape, generator=dg, device=device, dtype=dtype)
    else:
        k = torch.randn(shape, generator=g, dtype=torch.float32).to(dtype)
        v = torch.randn(shape, generator=g, dtype=torch.float32).to(dtype)
    q = torch.randn((config.batch_capacity, config.query_heads, config.head_dim), generator=g,
                    dtype=torch.float32).to(dtype)
    return q.to(device), k.to(device), v.to(device), table.to(device)


def make_csr_inputs(config, lengths, seed=17, device="cuda", dtype=None, pool_tokens=None,
                    device_pool=False):
    """CSR fixture (page_size 1): (q, k/v [pool, Hkv, D], kv_indptr [B+1], kv_indices [sum L]).

    Token slots are the first sum(L) entries of a seeded permutation of the pool.  With
    ``device_pool`` the (large) K/V pools are drawn by a seeded generator on ``device``.
    """
    torch = _torch()
    dtype = torch.bfloat16 if dtype is None else dtype
    g = torch.Generator().manual_seed(seed)
    total = sum(lengths)
    pool = max(1, total, pool_tokens or 0)
    indices = torch.randperm(pool, generator=g)[:total].to(torch.int32)
    indptr = torch.zeros(len(lengths) + 1, dtype=torch.int32)
    indptr[1:] = torch.cumsum(torch.tensor(lengths, dtype=torch.int64), 0).to(torch.int32)
    q = torch.randn((config.batch_capacity, config.query_heads, config.head_dim), generator=g,
                    dtype=torch.float32).to(dtype)
    shape = (pool, config.kv_heads, config.head_dim)
    if device_pool:
        dg = torch.Generator(device=device).manual_seed(seed + 1)
        k = torch.randn(shape, generator=dg, device=device, dtype=dtype)
        v = torch.randn(shape, generator=dg, device=device, dtype=dtype)
    else:
        k = torch.randn(shape, generator=g, dtype=torch.float32).to(dtype).to(device)
        v = torch.randn(shape, generator=g, dtype=torch.float32).to(dtype).to(device)
    return q.to(device), k, v, indptr.to(device), indices.to(device)


def update_plan(engine, lengths, splits=None):
    """Write lengths/splits/active into the engine's plan buffers (benchmarks/workloads.py:43-50)."""
    torch = _torch()
    p = engine.plan
    splits = split_hints(lengths, engine.config.max_splits) if splits is None else splits
    n = len(lengths)
    host_l = torch.zeros(engine.config.batch_capacity, dtype=torch.int32)
    host_s = torch.ones(engine.config.batch_capacity, dtype=torch.int32)
    host_l[:n] = torch.tensor(lengths, dtype=torch.int32)
    host_s[:n] = torch.tensor(splits, dtype=torch.int32)
    p.lengths.copy_(host_l)
    p.splits.copy_(host_s)
    p.active.fill_(n)


def algorithmic_bytes(lengths, config, kv_itemsize=2, q_itemsize=2, out_itemsize=2, csr=None):
    """Algorithmic HBM bytes of one decode-attention layer for the active batch:
    sum_r L_r*Hkv*D*2*s_kv + index bytes + B*Hq*D*(s_q + s_o).  Index bytes are 4 per token
    for CSR page 1, else 4 per page."""
    csr = config.page_size == 1 if csr is None else csr
    total = sum(lengths)
    kv = total * config.kv_heads * config.head_dim * 2 * kv_itemsize
    if csr:
        idx = 4 * total
    else:
        idx = 4 * sum(math.ceil(n / config.page_size) for n in lengths)
    qo = len(lengths) * config.query_heads * config.head_dim * (q_itemsize + out_itemsize)
    return kv + idx + qo
