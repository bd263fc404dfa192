"""ORACLE (test infrastructure only): FP32 paged GQA decode attention.

Restates src/sglang_decode/reference/attention.py:5-18 in numpy float32: for each
request with L > 0, gather K/V rows through the page table (token t lives at
physical page pages[r, t // page_size], slot t % page_size), upcast to float32,
repeat each KV head for its query-head group, softmax(q.k * scale) @ v.  L == 0
rows are zero.  A CSR adapter maps kv_indptr/kv_indices (page_size 1) onto the
same gather, which is what runtime/engine.py:54-61 feeds the kernel.

Also restates the per-split partial/LSE slots written by
src/sglang_decode/kernels/attention.py:81-84 so the attention kernel can be
checked before the merge.
"""
import numpy as np


def _f32(x):
    """Accept torch tensors (any device, bf16/fp16) or numpy arrays."""
    try:
        import torch
        if isinstance(x, torch.Tensor):
            return x.detach().to("cpu", torch.float32).numpy()
    except ImportError:
        pass
    return np.asarray(x, dtype=np.float32)


def _ints(x):
    try:
        import torch
        if isinstance(x, torch.Tensor):
            return x.detach().to("cpu", torch.int64).numpy()
    except ImportError:
        pass
    return np.asarray(x, dtype=np.int64)


def _gather_rows(k, v, tokens_phys, tokens_inner):
    return k[tokens_phys, tokens_inner], v[tokens_phys, tokens_inner]


def paged_attention(q, k, v, pages, lengths, page_size, scale=None):
    """reference/attention.py:5-18.  q [B,Hq,D], k/v [P,page,Hkv,D], pages [B,max_pages]."""
    q, k, v, pages = _f32(q), _f32(k), _f32(v), _ints(pages)
    d = q.shape[-1]
    scale = np.float32(d ** -0.5 if scale is None else scale)
    group = q.shape[1] // k.shape[2]
    out = np.zeros(q.shape, dtype=np.float32)
    for r, length in enumerate(lengths):
        length = int(length)
        if length == 0:
            continue
        token = np.arange(length)
        phys = pages[r, token // page_size]
        key, value = _gather_rows(k, v, phys, token % page_size)          # [L, Hkv, D]
        key = np.repeat(key, group, axis=1)                               # [L, Hq, D]
        value = np.repeat(value, group, axis=1)
        score = np.einsum("hd,thd->ht", q[r], key).astype(np.float32) * scale
        score = score - score.max(axis=-1, keepdims=True)
        prob = np.exp(score)
        prob /= prob.sum(axis=-1, keepdims=True)
        out[r] = np.einsum("ht,thd->hd", prob, value)
    return out


def paged_attention_threads(q, k, v, pages, lengths, page_size, scale=None, threads=1):
    """paged_attention with the requests spread over `threads` host threads, for timing
    the CPU baseline on every core: per request (longest first) the rows are gathered
    in their storage dtype and upcast to float32, each KV head repeated for its group,
    then softmax(q.k * scale) @ v -- reference/attention.py:5-18 step for step, in torch
    CPU float32 (its ops release the GIL; one intra-op thread per worker thread).
    q/k/v/pages: CPU tensors or arrays of the shapes of paged_attention."""
    import concurrent.futures

    import torch
    q, k, v = (x if isinstance(x, torch.Tensor) else torch.from_numpy(np.asarray(x)) for x in (q, k, v))
    pages = torch.as_tensor(_ints(pages))
    d = q.shape[-1]
    scale = d ** -0.5 if scale is None else float(scale)
    group = q.shape[1] // k.shape[2]
    out = torch.zeros(q.shape, dtype=torch.float32)

    def one(r):
        n = int(lengths[r])
        if n == 0:
            return
        token = torch.arange(n)
        phys, inner = pages[r, token // page_size], token % page_size
        key = k[phys, inner].float().repeat_interleave(group, dim=1)    # [L, Hq, D]
        value = v[phys, inner].float().repeat_interleave(group, dim=1)
        score = torch.einsum("hd,thd->ht", q[r].float(), key) * scale
        out[r] = torch.einsum("ht,thd->hd", torch.softmax(score, dim=-1), value)

    order = sorted(range(len(lengths)), key=lambda r: -int(lengths[r]))
    previous = torch.get_num_threads()
    torch.set_num_threads(1)
    try:
        with concurrent.futures.ThreadPoolExecutor(max(1, int(threads))) as pool:
            list(pool.map(one, order))
    finally:
        torch.set_num_threads(previous)
    return out.numpy()


def csr_attention(q, k, v, kv_indptr, kv_indices, lengths, scale=None):
    """CSR token-index form (page_size 1): k/v [tokens, Hkv, D]."""
    k, v = _f32(k), _f32(v)
    indptr, indices = _ints(kv_indptr), _ints(kv_indices)
    b = len(lengths)
    maxl = max([int(x) for x in lengths] + [1])
    pages = np.zeros((max(b, 1), maxl), dtype=np.int64)
    for r in range(b):
        n = int(lengths[r])
        pages[r, :n] = indices[indptr[r]:indptr[r] + n]
    return paged_attention(q, k[:, None], v[:, None], pages, lengths, 1, scale)


def split_partials(q, k, v, pages, lengths, page_size, records, hq, smax, scale=None):
    """Per-(request, head, split) normalized partial outputs and natural-log LSE,
    following kernels/attention.py:48-84 for every record (request, split, begin, end).
    Returns dict {(r, h, s): (partial[D], lse)}."""
    q, k, v, pages = _f32(q), _f32(k), _f32(v), _ints(pages)
    d = q.shape[-1]
    scale = np.float32(d ** -0.5 if scale is None else scale)
    hkv = k.shape[2]
    group = hq // hkv
    out = {}
    for (r, s, begin, end) in records:
        token = np.arange(begin, end)
        phys = pages[r, token // page_size]
        key, value = _gather_rows(k, v, phys, token % page_size)
        for h in range(hq):
            g = h // group
            score = (key[:, g] @ q[r, h]).astype(np.float32) * scale
            m = score.max()
            p = np.exp(score - m)
            den = p.sum()
            out[(r, h, s)] = ((p @ value[:, g]) / den, float(m + np.log(den)))
    return out
