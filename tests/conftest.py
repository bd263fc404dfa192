import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(ROOT, "-sglang-decode-_amd")
for path in (PKG_ROOT, ROOT):
    if path not in sys.path:
        sys.path.insert(0, path)


# The reference's tests import its FP32 oracle as sglang_decode.reference.attention and its
# harness as benchmarks.workloads.  Neither is part of the product package here: the
# stand-ins under tests/compat map them onto oracle/ and sglang_decode.workloads, and are
# registered under the reference's module names for the test session only.
COMPAT = os.path.join(ROOT, "tests", "compat")
if COMPAT not in sys.path:
    sys.path.insert(0, COMPAT)


def _register_reference_oracle():
    import importlib
    import types
    if "sglang_decode.reference.attention" in sys.modules:
        return
    import sglang_decode
    parent = types.ModuleType("sglang_decode.reference")
    parent.__path__ = []
    parent.__doc__ = "test-session alias package (tests/conftest.py)"
    shim = importlib.import_module("reference_attention")
    parent.attention = shim
    sys.modules["sglang_decode.reference"] = parent
    sys.modules["sglang_decode.reference.attention"] = shim
    sglang_decode.reference = parent


_register_reference_oracle()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def pytest_collection_modifyitems(config, items):
    have_gpu = False
    try:
        import torch
        have_gpu = torch.cuda.is_available()
    except Exception:
        pass
    if have_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def plan_vectors():
    import json
    with open(os.path.join(ROOT, "tests", "golden", "plan_vectors.json")) as f:
        return json.load(f)
