"""Split merge launch (kernel in csrc/merge.hip); kernels/merge.py:7-30 of the reference."""
from .. import _lib
from .._lib import check, ptr


def merge_splits(plan, layer, min_splits=1):
    """Every row's merge (min_splits 1, the reference's), or only the rows of requests
    with at least ``min_splits`` splits (the attention wrote the others, see
    kernels.attention.persistent_decode's ``out``); rows without splits are zeroed and a
    plan error writes NaN either way."""
    c = plan.config
    args = (ptr(layer.partial), ptr(layer.lse), ptr(plan.counts), ptr(plan.active), ptr(plan.error),
            ptr(layer.output), c.batch_capacity, c.query_heads, c.head_dim, c.max_splits)
    tail = (_lib.dtype_code(layer.output.dtype), _lib.stream_handle(layer.output.device))
    if min_splits <= 1:
        check(_lib.lib().sgd_merge_splits(*args, *tail), "merge_splits")
    else:
        check(_lib.lib().sgd_merge_splits_min(*args, int(min_splits), *tail), "merge_splits")
