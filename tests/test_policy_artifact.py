"""The MI355X policy artifact shipped in the package (sglang_decode/policies/mi355x.json):
it is the calibration gate's own output on the committed sample sets, it loads, its rules
pick the published dynamic schedules on the C2 and C3 shapes, and the uniform batch-1
step keeps the R1 bypass (kernels/plan.py:67-68) -- the plan's mode checked with the
oracle here, on the device in tests/test_gpu_policy.py.  Also the DECODE_POLICY meaning
of planning.policy.policy_from_env."""
import hashlib
import json

import pytest

from oracle import plan as OP
from sglang_decode import workloads as W
from sglang_decode.config import Mode
from sglang_decode.planning import calibrate as C
from sglang_decode.planning.policy import (POLICY_DIR, SHIPPED_POLICIES, load_policy, policy_from_env,
                                           shipped_policy)

from gpu_util import cfg_ns

ARTIFACT = SHIPPED_POLICIES["gfx950"]


def artifact():
    return json.loads(ARTIFACT.read_text())


def flat(rules):
    return [[r.min_tasks, r.max_tasks, r.min_ratio, r.max_ratio, r.mode] for r in rules]


def oracle_mode(name, lengths=None, workers=512):
    c = W.config_for(name, workers)
    lengths = W.lengths_for(name) if lengths is None else lengths
    splits = W.splits_for(name, lengths, c)
    n = len(lengths)
    lw = list(lengths) + [0] * (c.batch_capacity - n)
    sw = list(splits) + [1] * (c.batch_capacity - n)
    return OP.full_plan(lw, sw, n, cfg_ns(c), flat(load_policy(str(ARTIFACT))), -1)["mode"]


def test_artifact_is_the_gate_output_on_its_evidence(tmp_path):
    art = artifact()
    assert art["status"] == "validated" and len(art["evidence"]) == 4
    for e in art["evidence"]:
        assert hashlib.sha256((POLICY_DIR / e["path"]).read_bytes()).hexdigest() == e["sha256"]
    files = [POLICY_DIR / e["path"] for e in art["evidence"]]
    groups = [(files[2 * i], files[2 * i + 1], (r["min_tasks"], r["max_tasks"]), (r["min_ratio"], r["max_ratio"]))
              for i, r in enumerate(art["rules"])]
    redo = C.calibrate_rules(groups, tmp_path / "again.json")
    assert redo["rules"] == art["rules"]
    assert [r.mode for r in load_policy(str(ARTIFACT))] == [r["mode"] for r in art["rules"]]


def test_artifact_rules_pick_dynamic_schedules_and_keep_the_bypass():
    rules = artifact()["rules"]
    assert all(r["mode"] in (Mode.D1, Mode.D4) for r in rules)
    assert oracle_mode("c2") == rules[0]["mode"]  # 1776 tasks, weight ratio 200
    assert oracle_mode("c3") == rules[1]["mode"]  # 2032 tasks, weight ratio 400
    c5 = W.c5_lengths()
    assert oracle_mode("c5", c5[:1]) == Mode.R1   # uniform weights: the bypass
    assert oracle_mode("c5", c5[:17]) == Mode.R1  # 648 tasks: below every rule


def test_policy_from_env(tmp_path):
    assert policy_from_env(env={"DECODE_POLICY": "none"}) == []
    assert policy_from_env(env={"DECODE_POLICY": ""}) == []
    assert flat(policy_from_env(env={"DECODE_POLICY": str(ARTIFACT)})) == flat(load_policy(str(ARTIFACT)))
    # unset: the shipped artifact of the device; no GPU here, so none
    if shipped_policy() is None:
        assert policy_from_env(env={}) == []
    with pytest.raises(FileNotFoundError):
        policy_from_env(env={"DECODE_POLICY": str(tmp_path / "missing.json")})


def test_multi_rule_gate_publishes_all_or_nothing(tmp_path):
    def write(path, meds):
        lines = ["variant,trial,wall_us,status"]
        lines += [f"{k},{i},{m + 0.1 * i},ok" for k, m in meds.items() for i in range(5)]
        path.write_text("\n".join(lines) + "\n")
        return path
    win = dict(R1=100.0, STATIC_CPU=104.0, D1=90.0, D4=92.0)
    lose = dict(R1=100.0, STATIC_CPU=104.0, D1=99.0, D4=99.5)
    a, b = write(tmp_path / "a.csv", win), write(tmp_path / "b.csv", win)
    c_, d = write(tmp_path / "c.csv", win), write(tmp_path / "d.csv", lose)
    with pytest.raises(C.GateRejected):
        C.calibrate_rules([(a, b, (1, 10), (100, 200)), (c_, d, (1, 10), (201, 300))], tmp_path / "p.json")
    assert not (tmp_path / "p.json").exists()
    art = C.calibrate_rules([(a, b, (1, 10), (100, 200)), (a, b, (11, 20), (100, 200))], tmp_path / "p.json")
    assert [r["mode"] for r in art["rules"]] == [int(Mode.D1)] * 2 and len(art["evidence"]) == 4
    with pytest.raises(ValueError, match="weight ratio of at least 100"):
        C.calibrate_rules([(a, b, (1, 10), (50, 200))], tmp_path / "q.json")
