"""Offline calibration gate: freeze one bounded policy rule from two independent sets of
measured samples (calibration and holdout); runs no kernel.

Behaviour of scripts/calibrate_policy.py:10-59:
* a samples CSV has rows ``variant, wall_us, status`` (``bench.py --samples-csv`` writes
  them; extra columns are ignored).  Any row whose status is not ``ok`` is an error --
  failed samples are investigated, never dropped -- and each of R1, STATIC_CPU, D1, D4
  needs at least five samples;
* the candidate is the variant with the lowest median on the calibration set.  A dynamic
  candidate (D1/D4) must beat the better static variant (R1 or STATIC_CPU) by at least
  3% in median and with no overlap (its slowest sample faster than the static's
  fastest), else the static variant is taken;
* on the holdout set the candidate may not be more than 2% slower than the better
  static variant, and a dynamic candidate must be at least 3% faster there, again with no
  overlap -- otherwise nothing is published;
* a host-static (STATIC_CPU) winner is kept as the baseline and no rule is published for
  it (the device LPT is not substituted for it in AUTO);
* the artifact ``{"status": "validated", "evidence": [{path, sha256} x 2], "rules":
  [{min_tasks, max_tasks, min_ratio, max_ratio, mode}]}`` is created, never overwritten,
  and loads with ``planning.policy.load_policy``.

Usage: ``python -m sglang_decode.planning.calibrate CAL.csv HOLDOUT.csv --output
policy.json --tasks MIN MAX --ratio MIN MAX``.
"""
import argparse
import csv
import hashlib
import json
import statistics
from pathlib import Path

MODES = {"R1": 1, "STATIC_CPU": 2, "D1": 3, "D4": 4}
STATIC = ("R1", "STATIC_CPU")


class GateRejected(Exception):
    """The measurements do not support publishing a rule."""


def read_samples(path):
    groups = {}
    with Path(path).open(newline="") as f:
        for row in csv.DictReader(f):
            if row["status"] != "ok":
                raise ValueError("failed samples need investigation; do not silently drop them")
            groups.setdefault(row["variant"], []).append(float(row["wall_us"]))
    for name in MODES:
        if len(groups.get(name, [])) < 5:
            raise ValueError(f"at least five full-wall rounds required for {name}")
    return groups


def _median(groups, name):
    return statistics.median(groups[name])


def choose(calibration, holdout):
    """The variant the gate publishes (R1, D1 or D4); GateRejected when there is none."""
    static = min(STATIC, key=lambda n: _median(calibration, n))
    candidate = min(MODES, key=lambda n: _median(calibration, n))
    if candidate in ("D1", "D4"):
        gain = 1 - _median(calibration, candidate) / _median(calibration, static)
        if gain < 0.03 or max(calibration[candidate]) >= min(calibration[static]):
            candidate = static
    hold_static = min(STATIC, key=lambda n: _median(holdout, n))
    if _median(holdout, candidate) > 1.02 * _median(holdout, hold_static):
        raise GateRejected("holdout regression exceeds 2%; no policy published")
    if candidate in ("D1", "D4") and (_median(holdout, candidate) > 0.97 * _median(holdout, hold_static)
                                      or max(holdout[candidate]) >= min(holdout[hold_static])):
        raise GateRejected("dynamic holdout benefit is below the adoption gate")
    if candidate == "STATIC_CPU":
        raise GateRejected("host static wins: retain it as baseline; do not substitute GPU LPT in AUTO")
    return candidate


def calibrate(calibration_path, holdout_path, output, tasks, ratio):
    """Writes the validated artifact to ``output`` (which must not exist) and returns it."""
    calibration_path, holdout_path, output = Path(calibration_path), Path(holdout_path), Path(output)
    if calibration_path.resolve() == holdout_path.resolve():
        raise ValueError("independent holdout artifact required")
    candidate = choose(read_samples(calibration_path), read_samples(holdout_path))
    evidence = [dict(path=str(p), sha256=hashlib.sha256(p.read_bytes()).hexdigest())
                for p in (calibration_path, holdout_path)]
    artifact = dict(status="validated", evidence=evidence,
                    rules=[dict(min_tasks=int(tasks[0]), max_tasks=int(tasks[1]), min_ratio=int(ratio[0]),
                                max_ratio=int(ratio[1]), mode=MODES[candidate])])
    with output.open("x") as f:
        json.dump(artifact, f, indent=2)
    return artifact


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("calibration", type=Path)
    ap.add_argument("holdout", type=Path)
    ap.add_argument("--output", type=Path, required=True)
    ap.add_argument("--tasks", nargs=2, type=int, required=True)
    ap.add_argument("--ratio", nargs=2, type=int, required=True)
    args = ap.parse_args(argv)
    try:
        calibrate(args.calibration, args.holdout, args.output, args.tasks, args.ratio)
    except ValueError as e:
        ap.error(str(e))
    except GateRejected as e:
        raise SystemExit(str(e))


if __name__ == "__main__":
    main()
