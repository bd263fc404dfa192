"""Split merge launch (kernel in csrc/merge.hip); kernels/merge.py:7-30 of the reference."""
from .. import _lib
from .._lib import check, ptr


def merge_splits(plan, layer):
    c = plan.config
    check(_lib.lib().sgd_merge_splits(
        ptr(layer.partial), ptr(layer.lse), ptr(plan.counts), ptr(plan.active), ptr(plan.error),
        ptr(layer.output), c.batch_capacity, c.query_heads, c.head_dim, c.max_splits,
        _lib.dtype_code(layer.output.dtype), _lib.stream_handle(layer.output.device)),
        "merge_splits")
