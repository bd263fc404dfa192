"""The policy calibration gate (sglang_decode/planning/calibrate.py), after
scripts/calibrate_policy.py:10-59, on synthetic sample sets: each outcome of the gate --
publish a dynamic rule, fall back to R1, refuse on a holdout regression, on a dynamic
benefit below 3% or overlapping samples, on a host-static win -- plus the input checks
(failed samples, fewer than five rounds, the same file twice, an existing output) and the
artifact loading with load_policy."""
import csv
import json

import pytest

from sglang_decode.config import Mode
from sglang_decode.planning import calibrate as C
from sglang_decode.planning.policy import load_policy


def write(path, medians, spread=0.5, n=5, status="ok"):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["variant", "trial", "wall_us", "status"])
        w.writeheader()
        for name, m in medians.items():
            for i in range(n):
                w.writerow(dict(variant=name, trial=i, wall_us=m + spread * (i - n // 2), status=status))
    return path


def run(tmp_path, cal, hold, **kw):
    a = write(tmp_path / "cal.csv", cal, **kw)
    b = write(tmp_path / "hold.csv", hold, **kw)
    return C.calibrate(a, b, tmp_path / "policy.json", (1, 4096), (150, 10000))


def test_dynamic_winner_is_published_and_loads(tmp_path):
    meds = dict(R1=100.0, STATIC_CPU=104.0, D1=90.0, D4=92.0)
    art = run(tmp_path, meds, meds)
    assert art["status"] == "validated" and len(art["evidence"]) == 2
    assert art["rules"] == [dict(min_tasks=1, max_tasks=4096, min_ratio=150, max_ratio=10000, mode=3)]
    rules = load_policy(str(tmp_path / "policy.json"))
    assert rules[0].mode == Mode.D1
    assert all(len(e["sha256"]) == 64 for e in art["evidence"])


def test_small_or_overlapping_dynamic_gain_falls_back_to_r1(tmp_path):
    art = run(tmp_path, dict(R1=100.0, STATIC_CPU=105.0, D1=98.0, D4=99.0),
              dict(R1=100.0, STATIC_CPU=105.0, D1=98.0, D4=99.0))
    assert art["rules"][0]["mode"] == int(Mode.R1)  # 2% < 3%
    (tmp_path / "policy.json").unlink()
    art = run(tmp_path, dict(R1=100.0, STATIC_CPU=105.0, D1=96.0, D4=99.0),
              dict(R1=100.0, STATIC_CPU=105.0, D1=96.0, D4=99.0), spread=2.0)
    assert art["rules"][0]["mode"] == int(Mode.R1)  # 4% but the samples overlap


@pytest.mark.parametrize("hold,reason", [
    (dict(R1=100.0, STATIC_CPU=104.0, D1=99.0, D4=104.0), "does not repeat its gain"),    # 1% gain on the holdout
    (dict(R1=100.0, STATIC_CPU=96.0, D1=97.0, D4=104.0), "does not repeat its gain"),     # host static now faster
])
def test_holdout_rejects_dynamic(tmp_path, hold, reason):
    with pytest.raises(C.GateRejected, match=reason):
        run(tmp_path, dict(R1=100.0, STATIC_CPU=104.0, D1=90.0, D4=92.0), hold)
    assert not (tmp_path / "policy.json").exists()


def test_holdout_regression_and_host_static_win(tmp_path):
    with pytest.raises(C.GateRejected, match="more than 2% slower"):  # R1 chosen, 5% slower on holdout
        run(tmp_path, dict(R1=100.0, STATIC_CPU=104.0, D1=110.0, D4=111.0),
            dict(R1=105.0, STATIC_CPU=100.0, D1=110.0, D4=111.0))
    with pytest.raises(C.GateRejected, match="host LPT is fastest"):
        run(tmp_path, dict(R1=104.0, STATIC_CPU=100.0, D1=110.0, D4=111.0),
            dict(R1=104.0, STATIC_CPU=100.0, D1=110.0, D4=111.0))


def test_input_checks(tmp_path):
    meds = dict(R1=100.0, STATIC_CPU=104.0, D1=90.0, D4=92.0)
    with pytest.raises(ValueError, match="has to be explained"):
        run(tmp_path, meds, meds, status="timeout")
    with pytest.raises(ValueError, match="at least 5 samples"):
        run(tmp_path, meds, meds, n=4)
    a = write(tmp_path / "a.csv", meds)
    with pytest.raises(ValueError, match="independent file"):
        C.calibrate(a, a, tmp_path / "p.json", (1, 2), (100, 200))
    b = write(tmp_path / "b.csv", meds)
    (tmp_path / "p.json").write_text("{}")
    with pytest.raises(FileExistsError):  # an artifact is never overwritten
        C.calibrate(a, b, tmp_path / "p.json", (1, 2), (100, 200))
    assert json.loads((tmp_path / "p.json").read_text()) == {}


def test_command_line(tmp_path):
    meds = dict(R1=100.0, STATIC_CPU=104.0, D1=95.0, D4=90.0)
    a, b = write(tmp_path / "a.csv", meds), write(tmp_path / "b.csv", meds)
    C.main([str(a), str(b), "--output", str(tmp_path / "p.json"), "--tasks", "8", "512", "--ratio", "100", "400"])
    assert load_policy(str(tmp_path / "p.json"))[0].mode == Mode.D4
    with pytest.raises(SystemExit):
        C.main([str(a), str(a), "--output", str(tmp_path / "q.json"), "--tasks", "8", "512", "--ratio", "100", "400"])
