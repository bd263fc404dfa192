"""Host-side tests (no GPU): config and policy contracts, the host planning API
against the reference's golden sequences, the C++ host LPT planner, the C-ABI
library's exports, and the engine's host validation (ValueError before any launch)."""
import ctypes
import json
import os
import re
import types

import pytest

from sglang_decode.config import DecodeConfig, Mode
from sglang_decode.planning import reference as R
from sglang_decode.planning.policy import PolicyRule, load_policy
from sglang_decode import workloads as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


# ------------------------------------------------------------------ config / policy

def test_config_defaults_and_derived():
    c = DecodeConfig()
    assert (c.batch_capacity, c.max_splits, c.max_context, c.query_heads, c.kv_heads, c.head_dim,
            c.page_size, c.workers, c.block_kv, c.split_alignment) == (64, 16, 32768, 32, 8, 128, 16,
                                                                       108, 128, 32)
    assert c.group_size == 4 and c.record_capacity == 1024 and c.task_capacity == 8192
    assert c.max_pages == 2048 and c.buckets == 9
    assert W.config_for("c1").buckets == 2 and W.config_for("c2").buckets == 7
    assert W.config_for("c4").buckets == 8 and W.config_for("c4").max_pages == 1024


@pytest.mark.parametrize("kw", [dict(batch_capacity=0), dict(query_heads=24, kv_heads=8),
                                dict(query_heads=64, kv_heads=2), dict(head_dim=96),
                                dict(block_kv=64), dict(split_alignment=16),
                                dict(batch_capacity=1024, max_splits=32), dict(workers=5000)])
def test_config_rejects(kw):
    with pytest.raises(ValueError):
        DecodeConfig(**kw)


def test_config_lifts_reference_record_bound_for_c3():
    c = W.config_for("c3")
    assert c.record_capacity == 8192 and c.task_capacity == 65536


def test_policy_gate(tmp_path):
    assert load_policy() == []
    path = tmp_path / "p.json"
    path.write_text(json.dumps({"status": "unvalidated", "evidence": [], "rules": []}))
    with pytest.raises(ValueError):
        load_policy(path)
    path.write_text(json.dumps({"status": "validated", "evidence": [], "rules": []}))
    with pytest.raises(ValueError):
        load_policy(path)
    good = {"status": "validated", "evidence": [{"path": "x", "sha256": "0"}],
            "rules": [dict(min_tasks=1, max_tasks=100, min_ratio=101, max_ratio=900, mode=4)]}
    path.write_text(json.dumps(good))
    assert load_policy(path) == [PolicyRule(1, 100, 101, 900, 4)]
    for bad in (dict(mode=0), dict(min_ratio=99), dict(max_tasks=0), dict(min_tasks=-1)):
        row = dict(good["rules"][0], **bad)
        path.write_text(json.dumps(dict(good, rules=[row])))
        with pytest.raises(ValueError):
            load_policy(path)


# ------------------------------------------------------------------ host planning API

def _cfg(case):
    cc = case["config"]
    return types.SimpleNamespace(**cc)


def test_host_planning_matches_reference_sequences(plan_vectors):
    for case in plan_vectors:
        c = _cfg(case)
        records, counts, offsets = R.split_records(case["lengths"], case["splits"], c)
        assert [[r.request, r.split, r.begin, r.end, r.weight] for r in records] == case["records"]
        assert counts == case["counts"] and offsets == case["offsets"]
        order = R.bucket_order(records)
        assert order == case["order"], case["name"]
        assert [list(p) for p in R.make_packs(records, order, c.kv_heads, c.workers, 1)] == case["packs_d1"]
        assert [list(p) for p in R.make_packs(records, order, c.kv_heads, c.workers, 4)] == case["packs_d4"]
        assert R.greedy_static(records, c.kv_heads, c.workers) == case["static_lists"]
        R.validate_plan(records, order, R.make_packs(records, order, c.kv_heads, c.workers), c.kv_heads)


@pytest.mark.parametrize("lengths,splits", [([32769], [1]), ([1], [0]), ([1] * 65, [1] * 65)])
def test_host_capacity_rejected(lengths, splits):
    with pytest.raises(ValueError):
        R.split_records(lengths, splits, DecodeConfig())


def test_validate_plan_catches_duplicates():
    c = DecodeConfig()
    records, _, _ = R.split_records([300, 40], [2, 1], c)
    order = R.bucket_order(records)
    packs = R.make_packs(records, order, c.kv_heads, c.workers)
    R.validate_plan(records, order, packs, c.kv_heads)
    with pytest.raises(AssertionError):
        R.validate_plan(records, order, packs + [packs[0]], c.kv_heads)


def test_split_hints_rule():
    assert W.split_hints([512] * 24 + [8192] * 8) == [1] * 24 + [16] * 8
    assert W.split_hints([256] * 24 + [1536] * 4 + [16384] * 4) == [1] * 24 + [2] * 4 + [16] * 4
    assert W.split_hints([0, 0]) == [1, 1]


def test_seeded_workloads_are_deterministic():
    assert W.c2_lengths() == W.c2_lengths()
    c2 = W.c2_lengths()
    assert len(c2) == 64 and min(c2) >= 128 and max(c2) <= 8192
    c3 = W.c3_lengths()
    assert c3[:2] == [32768, 32768] and len(c3) == 128 and all(32 <= x <= 512 for x in c3[2:])
    c4 = W.c4_lengths()
    assert len(c4) == 32 and all(2048 <= x <= 16384 for x in c4)
    assert W.algorithmic_bytes([1000, 24], W.config_for("c2")) == (
        1024 * 8 * 128 * 2 * 2 + 4 * 1024 + 2 * 32 * 128 * 4)


# ------------------------------------------------------------------ native library

def _header_symbols():
    text = open(os.path.join(ROOT, "include", "sglang_decode_hip.h")).read()
    return sorted(set(re.findall(r"\b(sgd_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from sglang_decode import _lib
    handle = _lib.lib()
    symbols = _header_symbols()
    assert len(symbols) >= 10
    for name in symbols:
        assert hasattr(handle, name), name
    assert b"gfx950" in handle.sgd_version()


def test_struct_layouts_match_header(tmp_path):
    """Every ctypes field sits at the offset the C header gives it (gcc prints offsetof
    for each field of sgd_decode_args, sgd_plan_buffers and sgd_noalloc_args), and the sizes
    agree."""
    import shutil
    import subprocess
    from sglang_decode._lib import DecodeArgsC, NoAllocArgsC, PlanBuffersC
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    include = os.path.join(ROOT, "include")
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "sglang_decode_hip.h"', 'int main(void) {']
    for cstruct, pystruct in (("sgd_decode_args", DecodeArgsC), ("sgd_plan_buffers", PlanBuffersC),
                              ("sgd_noalloc_args", NoAllocArgsC)):
        lines.append(f'printf("{cstruct} size %zu\\n", sizeof({cstruct}));')
        for name, _ in pystruct._fields_:
            lines.append(f'printf("{cstruct} {name} %zu\\n", offsetof({cstruct}, {name}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run([gcc, "-I", include, str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = {tuple(line.split()[:2]): int(line.split()[2]) for line in out if line}
    for cstruct, pystruct in (("sgd_decode_args", DecodeArgsC), ("sgd_plan_buffers", PlanBuffersC),
                              ("sgd_noalloc_args", NoAllocArgsC)):
        assert got[(cstruct, "size")] == ctypes.sizeof(pystruct), cstruct
        for name, _ in pystruct._fields_:
            assert got[(cstruct, name)] == getattr(pystruct, name).offset, (cstruct, name)


def test_host_static_lists_cpp_matches_reference(plan_vectors):
    from sglang_decode import _lib
    lib = _lib.lib()
    for case in plan_vectors:
        c = _cfg(case)
        weights = [r[4] for r in case["records"]]
        n = len(weights)
        cap = c.batch_capacity * c.max_splits * c.kv_heads
        w = (ctypes.c_int32 * max(n, 1))(*weights)
        heads = (ctypes.c_int32 * c.workers)()
        nxt = (ctypes.c_int32 * cap)()
        assert lib.sgd_host_static_lists(w, n, c.kv_heads, c.workers, cap, heads, nxt) == 0
        lists = R.lists_to_links(case["static_lists"], c.workers, cap)
        assert list(heads) == lists[0] and list(nxt) == lists[1], case["name"]
        # the same lists from the plan inputs: records formed in C++ from lengths / splits
        if not case.get("lengths"):
            continue
        b = len(case["lengths"])
        ln = (ctypes.c_int32 * b)(*case["lengths"])
        sp = (ctypes.c_int32 * b)(*case["splits"])
        heads2, nxt2, count = (ctypes.c_int32 * c.workers)(), (ctypes.c_int32 * cap)(), ctypes.c_int32(-1)
        assert lib.sgd_host_static_plan(ln, sp, b, c.max_splits, c.max_context, c.block_kv, c.kv_heads, c.workers,
                                        cap, heads2, nxt2, ctypes.byref(count)) == 0, case["name"]
        assert count.value == n, case["name"]
        assert list(heads2) == lists[0] and list(nxt2) == lists[1], case["name"]


def test_host_static_plan_rejects_bad_inputs():
    """The C++ host planner refuses a length beyond max_context, a split count outside
    [1, max_splits] and more tasks than the capacity, with the request named."""
    from sglang_decode import _lib
    lib = _lib.lib()
    heads, nxt = (ctypes.c_int32 * 8)(), (ctypes.c_int32 * 64)()

    def run(lengths, splits, max_context=1024, cap=64):
        b = len(lengths)
        return lib.sgd_host_static_plan((ctypes.c_int32 * b)(*lengths), (ctypes.c_int32 * b)(*splits), b, 4,
                                        max_context, 128, 2, 8, cap, heads, nxt, None)

    assert run([100, 1024], [1, 4]) == 0
    assert run([100, 1025], [1, 4]) == -22 and b"request 1" in lib.sgd_last_error()
    assert run([100, -1], [1, 1]) == -22
    assert run([100], [0]) == -22 and run([100], [5]) == -22
    assert run([1024] * 9, [4] * 9) == -22 and b"task capacity" in lib.sgd_last_error()  # 36 records x 2 > 64


def test_abi_rejects_bad_arguments_before_launch():
    from sglang_decode import _lib
    lib = _lib.lib()
    assert lib.sgd_count_scan(None, None, None, None, None, None, None, None, 0, 16, 256, None) == -22
    assert b"bcap" in lib.sgd_last_error()
    args = _lib.DecodeArgsC()
    args.query_heads, args.kv_heads, args.head_dim = 32, 8, 96
    assert lib.sgd_persistent_decode(ctypes.byref(args), None) == -22
    with pytest.raises(ValueError):
        _lib.check(-22, "x")


def test_attention_kernel_selection_is_host_only():
    """sgd_attention_kernel answers from the arguments alone (no device access):
    forced kernels are validated against the geometry they need."""
    from sglang_decode import _lib
    lib = _lib.lib()
    args = _lib.DecodeArgsC()
    # fake, aligned, never-dereferenced addresses: the query reads no memory
    for name in ("q", "k", "v", "pages", "partial", "lse", "counter", "indptr"):
        setattr(args, name, 1 << 20)
    args.query_heads, args.kv_heads, args.head_dim = 32, 8, 128
    args.max_splits, args.page_size, args.csr, args.workers = 16, 1, 1, 256
    args.k_stride[:] = [1024, 0, 128, 1]
    args.v_stride[:] = [1024, 0, 128, 1]
    for forced in ("generic", "valu", "mfma"):
        args.kernel = _lib.KERNELS[forced]
        assert _lib.KERNEL_NAMES[lib.sgd_attention_kernel(ctypes.byref(args))] == forced
    # AUTO picks a bitwise-repeatable kernel whatever the worker count: VALU for group 4
    # with one worker per CU (the reference's convention) as with two
    args.kernel = _lib.KERNELS["auto"]
    for workers in (108, 256, 512):
        args.workers = workers
        assert _lib.KERNEL_NAMES[lib.sgd_attention_kernel(ctypes.byref(args))] == "valu"
    # paged with a page size that is not a power of two: still the tuned kernels
    args.csr, args.page_size = 0, 12
    args.k_stride[:] = [12 * 1024, 1024, 128, 1]
    args.v_stride[:] = [12 * 1024, 1024, 128, 1]
    assert _lib.KERNEL_NAMES[lib.sgd_attention_kernel(ctypes.byref(args))] == "valu"
    args.kernel = _lib.KERNELS["mfma"]
    assert _lib.KERNEL_NAMES[lib.sgd_attention_kernel(ctypes.byref(args))] == "mfma"
    args.kernel = _lib.KERNELS["auto"]
    args.csr, args.page_size = 1, 1
    args.k_stride[:] = [1024, 0, 128, 1]
    args.v_stride[:] = [1024, 0, 128, 1]
    args.query_heads = 64  # group 8: no VALU kernel, the MFMA one serves it
    assert _lib.KERNEL_NAMES[lib.sgd_attention_kernel(ctypes.byref(args))] == "mfma"
    args.kernel = _lib.KERNELS["valu"]
    assert lib.sgd_attention_kernel(ctypes.byref(args)) == -22
    assert b"group <= 4" in lib.sgd_last_error()
    args.kernel = _lib.KERNELS["mfma"]
    assert _lib.KERNEL_NAMES[lib.sgd_attention_kernel(ctypes.byref(args))] == "mfma"
    for d in (64, 256):  # group 8: the MFMA kernel at every head dim
        args.head_dim = d
        args.k_stride[:] = [8 * d, 0, d, 1]
        args.v_stride[:] = [8 * d, 0, d, 1]
        assert _lib.KERNEL_NAMES[lib.sgd_attention_kernel(ctypes.byref(args))] == "mfma"
        args.kernel = _lib.KERNELS["auto"]
        assert _lib.KERNEL_NAMES[lib.sgd_attention_kernel(ctypes.byref(args))] == "mfma"
        args.kernel = _lib.KERNELS["mfma"]
    args.k_stride[:] = [8 * 64 + 8, 0, 64, 2]  # a dim stride of 2: the generic kernel only
    args.v_stride[:] = [8 * 64 + 8, 0, 64, 2]
    args.head_dim = 64
    assert lib.sgd_attention_kernel(ctypes.byref(args)) == -22
    args.kernel = _lib.KERNELS["auto"]
    assert _lib.KERNEL_NAMES[lib.sgd_attention_kernel(ctypes.byref(args))] == "generic"
    args.query_heads = 32  # group 4: the VALU kernel at every head_dim
    for d in (64, 128, 256):
        args.head_dim = d
        args.k_stride[:] = [8 * d, 0, d, 1]
        args.v_stride[:] = [8 * d, 0, d, 1]
        assert _lib.KERNEL_NAMES[lib.sgd_attention_kernel(ctypes.byref(args))] == "valu"


# ------------------------------------------------------------------ engine host validation

def test_engine_validates_before_launch():
    import torch
    from sglang_decode.runtime.engine import DecodeEngine
    c = W.config_for("c1")
    engine = DecodeEngine(c, device="cpu", layers=1)
    q = torch.zeros(c.batch_capacity, c.query_heads, c.head_dim, dtype=torch.bfloat16)
    k = torch.zeros(10, 1, c.kv_heads, c.head_dim, dtype=torch.bfloat16)
    pages = torch.zeros(c.batch_capacity, c.max_pages, dtype=torch.int32)
    with pytest.raises(ValueError):
        engine.execute(q.float(), k, k, pages)
    with pytest.raises(ValueError):
        engine.execute(q[:2], k, k, pages)
    with pytest.raises(ValueError):
        engine.execute(q, k[:, :, :1], k[:, :, :1], pages)
    with pytest.raises(ValueError):
        engine.execute(q, k, k, pages[:, :3])
    with pytest.raises(ValueError):  # CSR needs 3-D KV
        engine.execute(q, k, k, pages.flatten(), indptr=torch.zeros(5, dtype=torch.int32))
    with pytest.raises(ValueError):  # index dtype
        engine.execute(q, k, k, pages.long())
    assert engine.plan.rules.tolist() == [[0, 0, 100, 100, 1]] and engine.plan.rule_count == 0
    assert engine.layers[0].partial.shape == (4, 8, 16, 128)
    assert engine.layers[0].lse.shape == (4, 8, 16)
    assert Mode.D4 == 4


def test_noalloc_wrapper_validates_before_launch():
    """decode_noalloc runs the engine's layout checks and sizes its plan inputs on the host:
    a short lengths/splits tensor, an int64 page table, mixed q/K dtypes, a wrong q shape or
    a mis-shaped out raise ValueError before the library is called (CPU tensors here)."""
    import torch
    from sglang_decode.kernels.noalloc import decode_noalloc
    c = W.config_for("c1")
    q = torch.zeros(c.batch_capacity, c.query_heads, c.head_dim, dtype=torch.bfloat16)
    k = torch.zeros(64, c.kv_heads, c.head_dim, dtype=torch.bfloat16)
    idx = torch.zeros(64, dtype=torch.int32)
    indptr = torch.zeros(c.batch_capacity + 1, dtype=torch.int32)
    lengths = torch.zeros(c.batch_capacity, dtype=torch.int32)
    active = torch.ones(1, dtype=torch.int32)
    out = torch.empty_like(q)

    def call(**kw):
        args = dict(q=q, k=k, v=k, pages=idx, lengths=lengths, splits=lengths.clone(), active=active, out=out,
                    indptr=indptr)
        args.update(kw)
        ip = args.pop("indptr")
        return decode_noalloc(c, **args, indptr=ip)

    for kw, what in ((dict(lengths=lengths[:2]), "lengths"), (dict(splits=lengths[:3].clone()), "splits"),
                     (dict(active=torch.ones(2, dtype=torch.int32)), "active"),
                     (dict(lengths=lengths.long()), "lengths"), (dict(pages=idx.long()), "int32"),
                     (dict(k=k.half(), v=k.half()), "dtype"), (dict(q=q[:2], out=out[:2]), "q must be"),
                     (dict(out=out[:, :, :64]), "out must be"), (dict(out=out.float()), "output"),
                     (dict(k=k[:, :1], v=k[:, :1]), "CSR K and V"),
                     (dict(indptr=indptr.long()), "kv_indptr")):
        with pytest.raises(ValueError, match=what):
            call(**kw)


def test_upstream_wrapper_validates_before_launch():
    """decode_attention_fwd checks the metadata sizes its stages index (kv_indptr[b + 1],
    num_kv_splits[b] for b < batch), K/V shape and dtype, and one device."""
    import torch
    from sglang_decode.kernels.upstream import decode_attention_fwd
    b, hq, hkv, d, s = 3, 8, 2, 128, 4
    q = torch.zeros(b, hq, d, dtype=torch.bfloat16)
    k = torch.zeros(32, hkv, d, dtype=torch.bfloat16)
    o = torch.empty_like(q)
    indptr = torch.zeros(b + 1, dtype=torch.int32)
    idx = torch.zeros(32, dtype=torch.int32)
    num = torch.ones(b, dtype=torch.int32)
    logits = torch.empty(b, hq, s, d)
    lse = torch.empty(b, hq, s)

    def call(**kw):
        args = dict(q=q, k_buffer=k, v_buffer=k, o=o, kv_indptr=indptr, kv_indices=idx, attn_logits=logits,
                    attn_lse=lse, num_kv_splits=num, max_kv_splits=s, sm_scale=0.1)
        args.update(kw)
        return decode_attention_fwd(**args)

    for kw, what in ((dict(kv_indptr=indptr[:b]), "kv_indptr"), (dict(num_kv_splits=num[:b - 1]), "num_kv_splits"),
                     (dict(k_buffer=k.half(), v_buffer=k.half()), "dtype"), (dict(k_buffer=k[0], v_buffer=k[0]),
                                                                              "k_buffer"),
                     (dict(v_buffer=k[:16]), "k_buffer"), (dict(kv_indptr=indptr.long()), "kv_indptr")):
        with pytest.raises(ValueError, match=what):
            call(**kw)


def test_host_static_schedule_installs_reference_lists(plan_vectors):
    """HostStatic (the benchmark's host-planned STATIC schedule) puts the reference's LPT
    lists into the plan and forces mode 2, with device ops only (here on a CPU plan)."""
    import torch
    from sglang_decode.planning.host_static import HostStatic
    from sglang_decode.runtime.engine import DecodeEngine
    case = next(c for c in plan_vectors if c["name"].startswith("B/"))
    cc = case["config"]
    c = DecodeConfig(batch_capacity=cc["batch_capacity"], max_splits=cc["max_splits"],
                     max_context=cc["max_context"], kv_heads=cc["kv_heads"],
                     query_heads=4 * cc["kv_heads"], workers=cc["workers"])
    engine = DecodeEngine(c, device="cpu", layers=1)
    hs = HostStatic(engine)
    hs.plan_lists(case["lengths"], case["splits"])
    hs.apply()
    heads, nxt = R.lists_to_links(case["static_lists"], c.workers, c.task_capacity)
    assert engine.plan.static_head.tolist() == heads
    assert engine.plan.static_next.tolist() == nxt
    assert engine.plan.mode.item() == 2
    with pytest.raises(ValueError):  # capacities are checked on the host
        hs.plan_lists([c.max_context + 1], [1])


def test_noalloc_rejects_geometry_beyond_its_scratch_before_any_device_call():
    """sgd_decode_noalloc's buffers must fit the library's 32 MiB array: batch 128 x 64
    splits x 32 heads x 128 dims of fp32 split slots (134 MB) is refused with the size
    needed, before the device is touched (this host has no GPU)."""
    from sglang_decode import _lib
    lib = _lib.lib()
    a = _lib.NoAllocArgsC()
    for name in ("q", "k", "v", "pages", "indptr", "lengths", "splits", "active", "out"):
        setattr(a, name, 1 << 20)
    a.batch_capacity, a.max_splits, a.max_context, a.workers = 128, 64, 32768, 512
    a.query_heads, a.kv_heads, a.head_dim, a.page_size, a.csr = 32, 8, 128, 1, 1
    assert lib.sgd_decode_noalloc(ctypes.byref(a), None) == -22
    msg = lib.sgd_last_error()
    assert b"needs" in msg and b"33554432" in msg
    # capacities whose products would overflow the size arithmetic are refused by bound
    for field, value in (("batch_capacity", 1 << 30), ("max_splits", 1 << 30), ("query_heads", 1 << 30),
                         ("head_dim", 1 << 20), ("workers", 1 << 30), ("kv_heads", 64)):
        saved = getattr(a, field)
        setattr(a, field, value)
        assert lib.sgd_decode_noalloc(ctypes.byref(a), None) == -22
        assert b"beyond the planner's bounds" in lib.sgd_last_error()
        setattr(a, field, saved)
    a.out = None
    assert lib.sgd_decode_noalloc(ctypes.byref(a), None) == -22
    assert b"null buffer" in lib.sgd_last_error()


def test_graph_update_checks_on_the_host():
    """DecodeGraph refuses a step that does not fit before touching any buffer: batch,
    context and split bounds, per-layer shapes, and in CSR mode kv_indices that hold
    fewer entries than the lengths need or more than the graph's capacity (the graph
    derives kv_indptr from the lengths itself, so the two cannot disagree)."""
    import torch
    from sglang_decode.runtime.engine import DecodeEngine, PlanKey
    from sglang_decode.runtime.graph import DecodeGraph
    c = DecodeConfig(batch_capacity=4, max_splits=4, max_context=256, page_size=1, workers=8)
    engine = DecodeEngine(c, device="cpu", layers=2)
    key = PlanKey("x", "hints", (32, 8, 128))
    kv = (torch.zeros(64, 8, 128, dtype=torch.bfloat16),) * 2
    with pytest.raises(ValueError, match="same plan key"):
        DecodeGraph(engine, [key, PlanKey("y", "hints", (32, 8, 128))], [kv] * 2, index_capacity=[64, 64])
    with pytest.raises(ValueError, match="capacities"):
        DecodeGraph(engine, [key] * 2, [kv] * 2, index_capacity=[64])
    graph = DecodeGraph(engine, [key] * 2, [kv] * 2, index_capacity=[64, 32])
    q = torch.zeros(2, 32, 128, dtype=torch.bfloat16)
    idx = torch.zeros(40, dtype=torch.int32)
    with pytest.raises(ValueError, match="batch 5"):
        graph.update([q] * 2, [idx] * 2, [1] * 5, [1] * 5)
    with pytest.raises(ValueError, match="context length"):
        graph.update([q] * 2, [idx] * 2, [10, 300], [1, 1])
    with pytest.raises(ValueError, match="split count"):
        graph.update([q] * 2, [idx] * 2, [10, 30], [1, 5])
    with pytest.raises(ValueError, match="layer 1 kv_indices has 40 entries; the step needs 40 and the graph "
                                         "holds 32"):
        graph.update([q] * 2, [idx] * 2, [10, 30], [1, 1])
    with pytest.raises(ValueError, match="step needs 50"):
        graph.update([q] * 2, [idx] * 2, [20, 30], [1, 1])
    with pytest.raises(ValueError, match="layer 0 q"):
        graph.update([q[:1]] * 2, [idx] * 2, [10, 30], [1, 1])
    with pytest.raises(RuntimeError, match="update"):
        graph.capture()


def test_upstream_comparator_rejects_bad_arguments_before_launch():
    """sgd_upstream_decode checks its geometry on the host (no GPU here): groups above 4,
    head_dim other than 128, K/V strides that are not multiples of 8, unaligned K/V."""
    from sglang_decode import _lib
    lib = _lib.lib()
    fake = ctypes.c_void_p(1 << 20)
    qs = (ctypes.c_int64 * 3)(4096, 128, 1)
    kvs = (ctypes.c_int64 * 4)(1024, 128, 1024, 128)

    def call(hq=32, hkv=8, d=128, strides=kvs, k=fake, batch=4):
        return lib.sgd_upstream_decode(fake, k, fake, fake, fake, fake, fake, fake, fake, batch, 16, hq, hkv, d, qs,
                                       strides, ctypes.c_float(0.1), 0, None)
    assert call(hq=64) == -22 and b"groups of up to 4" in lib.sgd_last_error()
    assert call(d=64) == -22 and b"head_dim" in lib.sgd_last_error()
    assert call(strides=(ctypes.c_int64 * 4)(1024, 127, 1024, 128)) == -22
    assert call(k=ctypes.c_void_p((1 << 20) + 8)) == -22 and b"aligned" in lib.sgd_last_error()
    assert call(batch=0) == 0  # nothing to do: no launch, no device access


def test_plan_entries_reject_unknown_forced_modes():
    """A forced mode outside R0..D4 is refused on the host (the device plan would otherwise
    take it as a schedule id)."""
    from sglang_decode import _lib
    from sglang_decode.runtime.workspace import PlanBuffers
    lib = _lib.lib()
    plan = PlanBuffers(W.config_for("c1"), "cpu")
    for bad in (-2, 5, 17):
        assert lib.sgd_build_plan(ctypes.byref(plan.c_struct()), bad, 0, None, 0, None) == -22
        assert b"force_mode" in lib.sgd_last_error()
        assert lib.sgd_order_and_packs(None, None, None, None, None, None, None, None, 0, bad, 2, 8, 2, 64,
                                       None) == -22
