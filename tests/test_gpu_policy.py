"""The shipped MI355X policy on the device: with DECODE_POLICY unset the adapter's rules
(planning.policy.policy_from_env) are the artifact for this GPU, and the device plan picks
the artifact's dynamic schedule at C2 and C3 and the R1 bypass for the uniform batch-1
step (kernels/plan.py:59-68)."""
import json

import pytest
import torch

from sglang_decode import workloads as W
from sglang_decode.config import Mode
from sglang_decode.planning.policy import SHIPPED_POLICIES, policy_from_env, shipped_policy
from sglang_decode.runtime.engine import DecodeEngine

pytestmark = pytest.mark.gpu


def picked(name, lengths, rules):
    c = W.config_for(name, 512)
    engine = DecodeEngine(c, layers=1, rules=rules)
    W.update_plan(engine, lengths, W.splits_for(name, lengths, c))
    engine.prepare()
    torch.cuda.synchronize()
    assert int(engine.plan.error.item()) == 0
    return int(engine.plan.mode.item())


def test_shipped_policy_picks_on_the_device():
    arch = torch.cuda.get_device_properties(0).gcnArchName.split(":")[0]
    if arch not in SHIPPED_POLICIES:
        pytest.skip(f"no policy artifact ships for {arch}")
    assert shipped_policy() == str(SHIPPED_POLICIES[arch])
    rules = policy_from_env(env={})
    published = [r["mode"] for r in json.loads(SHIPPED_POLICIES[arch].read_text())["rules"]]
    assert [int(r.mode) for r in rules] == published
    assert picked("c2", W.lengths_for("c2"), rules) == published[0]
    assert picked("c3", W.lengths_for("c3"), rules) == published[1]
    assert picked("c5", W.c5_lengths()[:1], rules) == Mode.R1
    assert picked("c2", W.lengths_for("c2"), policy_from_env(env={"DECODE_POLICY": "none"})) == Mode.R1
