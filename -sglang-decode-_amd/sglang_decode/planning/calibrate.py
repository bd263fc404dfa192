"""Policy calibration gate: turns two independent sets of measured step times into at
most one validated policy rule.  No kernel runs here.

The decision rules are the reference's (scripts/calibrate_policy.py:10-59); the code
and messages are this package's:

* Inputs are two CSV files (calibration, holdout) with columns ``variant``, ``wall_us``
  and ``status`` (``bench.py --samples-csv`` writes them; other columns are ignored).
  A row whose status is not ``ok`` stops the gate, and every schedule of the gate
  (R1, STATIC_CPU, D1, D4) needs five or more samples in each file.
* The pick is the schedule with the lowest calibration median.  A dynamic pick (D1/D4)
  stands only if it clears the bar against the better static schedule (R1 or
  STATIC_CPU): a median at least 3% lower and every sample below the static one's
  fastest.  Otherwise the static schedule is the pick.
* On the holdout set the pick may be at most 2% slower than the better static schedule
  there, and a dynamic pick must clear the same bar again; else nothing is published.
* A host-LPT pick (STATIC_CPU) is never published: it stays the baseline, and the device
  LPT is not put in its place.
* The artifact -- ``{"status": "validated", "evidence": [{path, sha256}, ...], "rules":
  [{min_tasks, max_tasks, min_ratio, max_ratio, mode}]}`` -- is written only to a path
  that does not exist yet, and ``planning.policy.load_policy`` reads it.
* Several shapes may share one artifact: each ``--rule`` names its own calibration and
  holdout files and the task / weight-ratio ranges its rule covers, every one passes the
  gate on its own files, and the artifact is written only when all of them pass (rules in
  the order given; the device plan lets the last matching rule win).

Usage: ``python -m sglang_decode.planning.calibrate CAL.csv HOLDOUT.csv --output
policy.json --tasks MIN MAX --ratio MIN MAX``, or ``... --output policy.json --rule CAL.csv
HOLDOUT.csv TASKS_MIN TASKS_MAX RATIO_MIN RATIO_MAX [--rule ...]``.
"""
import argparse
import csv
import hashlib
import json
import statistics
from pathlib import Path

from ..config import Mode

# Sample names of the gate and the device mode each one publishes.
SCHEDULES = {"R1": Mode.R1, "STATIC_CPU": Mode.STATIC, "D1": Mode.D1, "D4": Mode.D4}
STATIC = ("R1", "STATIC_CPU")
MIN_SAMPLES = 5
DYNAMIC_GAIN = 0.03      # a dynamic schedule's median must be this much below the static one
HOLDOUT_SLACK = 0.02     # how much slower than the best static schedule the pick may be on the holdout


class GateRejected(Exception):
    """The measurements do not support publishing a rule."""


class Samples:
    """Step times per schedule from one CSV file."""

    def __init__(self, path):
        self.path = Path(path)
        self.times = {}
        with self.path.open(newline="") as f:
            for line, row in enumerate(csv.DictReader(f), start=2):
                if row["status"] != "ok":
                    raise ValueError(f"{self.path}:{line}: sample status {row['status']!r}; a failed "
                                     "measurement has to be explained, not filtered out")
                self.times.setdefault(row["variant"], []).append(float(row["wall_us"]))
        short = [f"{name} ({len(self.times.get(name, []))})" for name in SCHEDULES
                 if len(self.times.get(name, [])) < MIN_SAMPLES]
        if short:
            raise ValueError(f"{self.path}: the gate needs at least {MIN_SAMPLES} samples per schedule; "
                             f"too few for {', '.join(short)}")

    def median(self, name):
        return statistics.median(self.times[name])

    def fastest(self, names):
        return min(names, key=self.median)

    def clears(self, dynamic, static):
        """True when ``dynamic`` beats ``static`` by the adoption bar: a median at least
        DYNAMIC_GAIN lower and no overlap (its slowest sample below the static's fastest)."""
        gain = 1.0 - self.median(dynamic) / self.median(static)
        return gain >= DYNAMIC_GAIN and max(self.times[dynamic]) < min(self.times[static])


def choose(calibration: Samples, holdout: Samples):
    """The schedule the gate publishes (R1, D1 or D4); GateRejected when there is none."""
    base = calibration.fastest(STATIC)
    pick = calibration.fastest(SCHEDULES)
    if pick not in STATIC and not calibration.clears(pick, base):
        pick = base
    hold_base = holdout.fastest(STATIC)
    if holdout.median(pick) > (1.0 + HOLDOUT_SLACK) * holdout.median(hold_base):
        raise GateRejected(f"{pick} is more than 2% slower than {hold_base} on the holdout set; "
                           "no rule published")
    if pick not in STATIC and not holdout.clears(pick, hold_base):
        raise GateRejected(f"{pick} does not repeat its gain over {hold_base} on the holdout set; "
                           "no rule published")
    if pick == "STATIC_CPU":
        raise GateRejected("the host LPT is fastest: it stays the baseline and "
                           "no device rule replaces it")
    return pick


def calibrate(calibration_path, holdout_path, output, tasks, ratio):
    """Writes the validated one-rule artifact to ``output`` (which must not exist) and
    returns it."""
    return calibrate_rules([(calibration_path, holdout_path, tasks, ratio)], output)


def calibrate_rules(groups, output):
    """``groups``: (calibration path, holdout path, (min_tasks, max_tasks), (min_ratio,
    max_ratio)) per rule.  Every group must pass the gate; then the artifact with one rule
    per group (in order) is written to ``output`` (which must not exist) and returned."""
    output = Path(output)
    if not groups:
        raise ValueError("no rule to calibrate")
    rules, files = [], []
    for cal, hold, tasks, ratio in groups:
        cal_path, hold_path = Path(cal), Path(hold)
        if cal_path.resolve() == hold_path.resolve():
            raise ValueError("the holdout set must be an independent file, not the calibration set")
        if not (0 <= int(tasks[0]) <= int(tasks[1]) and 100 <= int(ratio[0]) <= int(ratio[1])):
            raise ValueError(f"rule ranges tasks {tuple(tasks)} / ratio {tuple(ratio)}: need 0 <= min <= max "
                             "and a weight ratio of at least 100")
        pick = choose(Samples(cal_path), Samples(hold_path))
        rules.append(dict(min_tasks=int(tasks[0]), max_tasks=int(tasks[1]), min_ratio=int(ratio[0]),
                          max_ratio=int(ratio[1]), mode=int(SCHEDULES[pick])))
        files += [cal_path, hold_path]
    artifact = dict(status="validated",
                    evidence=[dict(path=str(p), sha256=hashlib.sha256(p.read_bytes()).hexdigest())
                              for p in files],
                    rules=rules)
    with output.open("x") as f:  # never replace an existing artifact
        json.dump(artifact, f, indent=2)
    return artifact


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("calibration", type=Path, nargs="?")
    ap.add_argument("holdout", type=Path, nargs="?")
    ap.add_argument("--output", type=Path, required=True)
    ap.add_argument("--tasks", nargs=2, type=int, metavar=("MIN", "MAX"))
    ap.add_argument("--ratio", nargs=2, type=int, metavar=("MIN", "MAX"))
    ap.add_argument("--rule", nargs=6, action="append", default=[],
                    metavar=("CAL", "HOLDOUT", "TASKS_MIN", "TASKS_MAX", "RATIO_MIN", "RATIO_MAX"))
    args = ap.parse_args(argv)
    single = (args.calibration, args.holdout, args.tasks, args.ratio)
    if args.rule and any(x is not None for x in single):
        ap.error("give either CAL HOLDOUT --tasks --ratio or --rule groups, not both")
    if not args.rule and any(x is None for x in single):
        ap.error("CAL, HOLDOUT, --tasks and --ratio are required without --rule")
    groups = [(args.calibration, args.holdout, args.tasks, args.ratio)] if not args.rule else [
        (Path(r[0]), Path(r[1]), (int(r[2]), int(r[3])), (int(r[4]), int(r[5]))) for r in args.rule]
    try:
        calibrate_rules(groups, args.output)
    except ValueError as e:
        ap.error(str(e))
    except GateRejected as e:
        raise SystemExit(str(e))


if __name__ == "__main__":
    main()
