"""Test-side stand-in for the reference's ``sglang_decode.reference.attention`` (its FP32
oracle, reference/attention.py:5-18), registered under that module name by
tests/conftest.py.  The oracle itself is oracle/attention.py; this returns its result as
a float32 torch tensor on the CPU, as the reference's function does."""
import torch

from oracle import attention as _oracle


def paged_attention(q, k, v, pages, lengths, page_size, scale=None):
    return torch.from_numpy(_oracle.paged_attention(q, k, v, pages, lengths, page_size, scale))
