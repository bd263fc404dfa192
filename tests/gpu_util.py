"""Helpers shared by the GPU tests: device plan read-back and oracle comparison."""
import types

import numpy as np
import torch

from oracle import plan as OP


def cfg_ns(c):
    return types.SimpleNamespace(batch_capacity=c.batch_capacity, max_splits=c.max_splits,
                                 max_context=c.max_context, workers=c.workers,
                                 kv_heads=c.kv_heads, block_kv=c.block_kv)


def read_plan(plan):
    torch.cuda.synchronize()
    get = lambda t: t.cpu().tolist()
    return {k: get(getattr(plan, k)) for k in (
        "counts", "offsets", "chunk", "request", "split", "begin", "end", "weight", "order",
        "pack_first", "pack_count", "static_head", "static_next")} | {
        k: int(getattr(plan, k).item()) for k in ("record_count", "num_packs", "mode", "error")}


def assert_plan_equal(dev, ref, config, active, name=""):
    """Bit-exact comparison of the device plan with oracle.full_plan."""
    b = config.batch_capacity
    assert dev["error"] == ref["error"], name
    assert dev["record_count"] == ref["record_count"], name
    assert dev["counts"][:b] == ref["counts"], name
    assert dev["offsets"][:b + 1] == ref["offsets"], name
    assert dev["chunk"][:b] == ref["chunk"], name
    assert dev["mode"] == ref["mode"], name
    assert dev["num_packs"] == ref["num_packs"], name
    n = ref["record_count"]
    if "request" in ref:
        for k in ("request", "split", "begin", "end", "weight"):
            assert dev[k][:n] == ref[k][:n], (name, k)
        assert dev["order"][:n] == ref["order"], name
        npk = ref["num_packs"]
        assert dev["pack_first"][:npk] == ref["pack_first"], name
        assert dev["pack_count"][:npk] == ref["pack_count"], name
    if ref.get("static_head") is not None and ref["mode"] == 2:
        assert OP.walk_lists(dev["static_head"], dev["static_next"]) == \
            OP.walk_lists(ref["static_head"], ref["static_next"]), name


def close(actual, expected, atol=2e-2, rtol=1e-2, msg=""):
    """The path's tolerance for bf16/fp16 inputs vs the FP32 oracle: 2e-2 abs / 1e-2 rel."""
    a = actual.float().cpu().numpy() if isinstance(actual, torch.Tensor) else np.asarray(actual)
    np.testing.assert_allclose(a, expected, atol=atol, rtol=rtol, err_msg=msg)
