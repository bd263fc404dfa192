"""ctypes binding of the C ABI in include/sglang_decode_hip.h.

The library is loaded after ``import torch`` so that it binds to the HIP runtime
torch already loaded (both use the SONAME libamdhip64.so.7): streams and device
pointers from torch are then valid in the library.  There is no fallback: if the
library is missing, every entry raises.
"""
import ctypes
import os

import torch  # noqa: F401  (must precede the library load, see above)

from ._build import LIB_PATH

SGD_EINVAL = -22
SGD_BF16, SGD_FP16 = 0, 1
KERNELS = {"auto": 0, "generic": 1, "valu": 2, "mfma": 3}
KERNEL_NAMES = {v: k for k, v in KERNELS.items()}

_P = ctypes.c_void_p
_I = ctypes.c_int32


class PlanBuffersC(ctypes.Structure):
    _fields_ = [(name, _P) for name in (
        "lengths", "splits", "active", "counts", "offsets", "chunk", "request", "split", "begin",
        "end", "weight", "order", "pack_first", "pack_count", "record_count", "num_packs", "mode",
        "error", "static_head", "static_next", "rules", "dispatch")] + [
        (name, _I) for name in ("rule_count", "batch_capacity", "max_splits", "max_context",
                                "kv_heads", "workers", "block_kv", "buckets")]


class DecodeArgsC(ctypes.Structure):
    _fields_ = [(name, _P) for name in (
        "q", "k", "v", "pages", "indptr", "lengths", "request", "split", "begin", "end", "order",
        "offsets", "chunk", "active", "record_count", "mode", "pack_first", "pack_count",
        "num_packs", "counter", "done_counter", "static_head", "static_next", "partial", "lse",
        "dispatch")] + [
        ("scale", ctypes.c_float), ("_pad0", _I),
        ("q_stride", ctypes.c_int64 * 3), ("k_stride", ctypes.c_int64 * 4),
        ("v_stride", ctypes.c_int64 * 4), ("pt_stride", ctypes.c_int64 * 2)] + [
        (name, _I) for name in ("query_heads", "kv_heads", "head_dim", "max_splits", "page_size",
                                "csr", "dtype", "workers", "kernel", "dispatch_units", "_pad1")] + [
        ("out", _P)]


class NoAllocArgsC(ctypes.Structure):
    _fields_ = [(name, _P) for name in ("q", "k", "v", "pages", "indptr", "lengths", "splits", "active", "out")] + [
        ("scale", ctypes.c_float), ("_pad0", _I),
        ("q_stride", ctypes.c_int64 * 3), ("k_stride", ctypes.c_int64 * 4),
        ("v_stride", ctypes.c_int64 * 4), ("pt_stride", ctypes.c_int64 * 2)] + [
        (name, _I) for name in ("batch_capacity", "max_splits", "max_context", "query_heads", "kv_heads",
                                "head_dim", "page_size", "csr", "dtype", "workers", "force_mode", "kernel")]


_SIGNATURES = {
    "sgd_last_error": (ctypes.c_char_p, []),
    "sgd_version": (ctypes.c_char_p, []),
    "sgd_count_scan": (_I, [_P] * 8 + [_I] * 3 + [_P]),
    "sgd_emit_records": (_I, [_P] * 9 + [_I] * 3 + [_P]),
    "sgd_order_and_packs": (_I, [_P] * 7 + [_P, _I, _I, _I, _I, _I, _I, _P]),
    "sgd_greedy_lists": (_I, [_P] * 5 + [_I] * 3 + [_P]),
    "sgd_build_plan": (_I, [ctypes.POINTER(PlanBuffersC), _I, _I, _P, _I, _P]),
    "sgd_build_plan_csr": (_I, [ctypes.POINTER(PlanBuffersC), _P, _P, _I, _I, _I, _P, _I, _P]),
    "sgd_csr_metadata": (_I, [_P, _I, _P, _I, _P, ctypes.c_int64, ctypes.c_int64, _I, _I, _I, _P, _P,
                              ctypes.c_int64, _P, _P, _P, _P, _P, _P]),
    "sgd_persistent_decode": (_I, [ctypes.POINTER(DecodeArgsC), _P]),
    "sgd_attention_kernel": (_I, [ctypes.POINTER(DecodeArgsC)]),
    "sgd_merge_splits": (_I, [_P] * 6 + [_I] * 5 + [_P]),
    "sgd_merge_splits_min": (_I, [_P] * 6 + [_I] * 6 + [_P]),
    "sgd_host_static_lists": (_I, [_P, _I, _I, _I, _I, _P, _P]),
    "sgd_host_static_plan": (_I, [_P, _P] + [_I] * 7 + [_P, _P, _P]),
    "sgd_decode_noalloc": (_I, [ctypes.POINTER(NoAllocArgsC), _P]),
    "sgd_upstream_decode": (_I, [_P] * 9 + [_I] * 5 + [_P, _P, ctypes.c_float, _I, _P]),
    "sgd_store_kv_stage_q": (_I, [_P, _P, _P, _P, _I, _P, _P, _P, ctypes.c_int64, _P, _P, _P, _P,
                                  _I, _I, _I, _I, _I, _P]),
}

_lib = None


def lib():
    """The loaded library; raises RuntimeError when it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"sglang_decode native library missing ({LIB_PATH}); build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` from the repository root")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(rc, what):
    if rc == 0:
        return
    msg = lib().sgd_last_error().decode(errors="replace")
    if rc == SGD_EINVAL:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what} failed (hipError {rc}): {msg}")


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_handle(device=None):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def dtype_code(dtype):
    if dtype == torch.bfloat16:
        return SGD_BF16
    if dtype == torch.float16:
        return SGD_FP16
    raise ValueError(f"unsupported dtype {dtype}")
