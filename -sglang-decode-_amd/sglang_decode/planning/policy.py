"""Policy files: which schedule the device plan picks for a batch's shape.

A policy file is the JSON artifact of the calibration gate (planning/calibrate.py), in
the format of src/sglang_decode/planning/policy.py:7-28: ``{"status": "validated",
"evidence": [...], "rules": [{min_tasks, max_tasks, min_ratio, max_ratio, mode}]}``.
Without a policy the plan runs R1.  A file must say it was validated and carry its
evidence; rules may select R1, STATIC, D1 or D4 over task-count and weight-ratio ranges
(the device plan lets the last matching rule win).

The package ships validated artifacts per GPU architecture (``policies/``, with the
sample sets they were calibrated on): ``shipped_policy`` finds the one for a device, and
``policy_from_env`` gives the adapter's ``DECODE_POLICY`` meaning -- unset: the shipped
artifact of the device (R1 where none ships); empty or ``none``: no rules, R1 (the
reference's default); otherwise the file it names.
"""
import json
import os
from dataclasses import dataclass
from pathlib import Path

from ..config import Mode

POLICY_DIR = Path(__file__).resolve().parent.parent / "policies"
# Validated artifacts by gfx architecture (the part of gcnArchName before any ':').
SHIPPED_POLICIES = {"gfx950": POLICY_DIR / "mi355x.json"}


@dataclass(frozen=True)
class PolicyRule:
    min_tasks: int
    max_tasks: int
    min_ratio: int  # max/min loop count, ratio scaled by 100
    max_ratio: int
    mode: int


_SELECTABLE = (Mode.R1, Mode.STATIC, Mode.D1, Mode.D4)


def load_policy(path=None):
    """The rules of a validated policy file, or [] without one (ValueError otherwise)."""
    if path is None:
        return []
    with open(path, encoding="utf-8") as f:
        artifact = json.load(f)
    if artifact.get("status") != "validated":
        raise ValueError(f"load_policy: {path} is not marked validated; only a calibrated artifact may "
                         "switch schedules")
    if not artifact.get("evidence"):
        raise ValueError(f"load_policy: {path} carries no calibration evidence")
    rules = []
    for i, row in enumerate(artifact["rules"]):
        rule = PolicyRule(**row)
        if rule.mode not in _SELECTABLE:
            raise ValueError(f"load_policy: rule {i} selects mode {rule.mode}; a rule may select R1, STATIC, "
                             "D1 or D4")
        if not 0 <= rule.min_tasks <= rule.max_tasks or rule.min_ratio < 100:
            raise ValueError(f"load_policy: rule {i} has empty or negative task bounds, or a weight ratio "
                             "below 100 (max/min x 100 is at least 100)")
        rules.append(rule)
    return rules


def shipped_policy(device=None):
    """Path of the validated artifact shipped for ``device``'s architecture, or None (no GPU,
    or an architecture nothing was calibrated on)."""
    import torch
    if not torch.cuda.is_available():
        return None
    dev = torch.device(device if device is not None else "cuda")
    if dev.type != "cuda":
        return None
    arch = torch.cuda.get_device_properties(dev).gcnArchName.split(":")[0]
    path = SHIPPED_POLICIES.get(arch)
    return str(path) if path is not None and path.exists() else None


def policy_from_env(device=None, env=None):
    """The rules ``DECODE_POLICY`` selects: unset -> the shipped artifact for ``device``
    ([] where none ships); "" or "none" -> []; otherwise load_policy of the path."""
    value = (os.environ if env is None else env).get("DECODE_POLICY")
    if value is None:
        return load_policy(shipped_policy(device))
    if value.strip().lower() in ("", "none"):
        return []
    return load_policy(value)
