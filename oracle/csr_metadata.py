"""ORACLE (test infrastructure only): the decode step's CSR metadata from the request pool.

Restates what the reference adapter consumes (src/sglang_decode/integrations/
sglang_backend.py:98-107: forward_metadata.kv_indptr / kv_indices / num_kv_splits), as
upstream SGLang v0.4.6.post5 (not vendored in the reference) produces it in its triton
backend's decode metadata hook: kv_indptr = [0, cumsum(seq_lens)], and kv_indices the
rows req_to_token[req_pool_indices[i], :seq_lens[i]] back to back (its
create_flashinfer_kv_indices_triton).  Split counts follow the reference harness rule,
benchmarks/workloads.py:20-21 (chunk = max(1, ceil(max L / S)), S_i = clamp(ceil(L_i /
chunk), 1, S)).  Invalid rows (negative, longer than a table row, pool index outside the
table) count as length 0 and set error; a valid total above the capacity makes every row
length 0 and sets error -- the rule of the HIP kernel, which must never read or write out
of bounds (upstream would index out of range instead).
"""
import math

import numpy as np


def harness_splits(lengths, maximum):
    """benchmarks/workloads.py:20-21."""
    chunk = max(1, math.ceil(max(lengths, default=0) / maximum))
    return [max(1, min(maximum, math.ceil(n / chunk))) for n in lengths]


def csr_metadata(seq_lens, req_pool_indices, req_to_token, max_splits, capacity):
    """Returns dict(kv_indptr [B+1], kv_indices [sum L], num_kv_splits [B], lengths [B],
    error 0/1), all plain int lists."""
    seq_lens = [int(x) for x in np.asarray(seq_lens).reshape(-1)]
    pool = [int(x) for x in np.asarray(req_pool_indices).reshape(-1)]
    table = np.asarray(req_to_token)
    rows, cols = table.shape
    lengths, error = [], 0
    for L, p in zip(seq_lens, pool):
        ok = 0 <= L <= cols and 0 <= p < rows
        lengths.append(L if ok else 0)
        error |= int(not ok and L != 0)
    if sum(lengths) > capacity:
        lengths, error = [0] * len(lengths), 1
    indptr = [0]
    indices = []
    for L, p in zip(lengths, pool):
        indptr.append(indptr[-1] + L)
        indices.extend(int(x) for x in table[p, :L]) if L else None
    return dict(kv_indptr=indptr, kv_indices=indices, num_kv_splits=harness_splits(lengths, max_splits),
                lengths=lengths, error=error)
