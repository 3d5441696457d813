"""Measure how far the oracle is from the reference's own output on every golden
case and write the per-case budgets the CPU tests hold it to.

The reference's fp32 reductions (torch CPU's mean / norm / amax order) are not
the oracle's canonical order, so a few elements of a golden case may differ.
This script replays every case through the oracle (tests/golden_compare.py)
against the fixtures under tests/golden/ and records, per case, exactly how
many elements differ and by how much; tests/test_oracle_golden.py then fails if
any count or distance grows.  Run from the repository root:

    python tests/golden/measure_budgets.py        # writes tests/golden/oracle_budgets.json

It reads only the committed fixtures and the oracle; it does not import the
reference.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

from golden_compare import CASES, CFG0, bf16_mismatch, build_oracle, load_golden, rel_err, run_oracle, set_grads  # noqa: E402

import oracle as O  # noqa: E402

_MOM = ("m", "m_pos", "m_neg")


def f32_ulps(a: np.ndarray, b: np.ndarray) -> int:
    """Largest distance between two fp32 arrays in units in the last place
    (consecutive floats are 1 apart on the monotone integer line)."""
    a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(b, dtype=np.float32).reshape(-1).view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return int(np.abs(a - b).max()) if a.size else 0


def bit_case(name: str) -> dict:
    """bf16-grad cases: weights, eval weights, momentum codes, scales, fp32 state."""
    case = CASES[name]
    gold = load_golden(name)
    params, _opt, evalp = run_oracle(case)
    out = {"kind": "bf16", "weights_total": 0, "weights_differ": 0, "weights_max_ulp": 0, "codes_differ": 0,
           "codes_total": 0, "scale_max_ulp": 0, "state_max_rel": 0.0}
    for i, prm in enumerate(params):
        nm, mu = bf16_mismatch(prm.p, gold[f"p{i}"])
        out["weights_total"] += int(prm.p.size)
        out["weights_differ"] += nm
        out["weights_max_ulp"] = max(out["weights_max_ulp"], mu)
        if evalp is not None:
            nm, mu = bf16_mismatch(evalp[i], gold[f"p{i}_eval"])
            out["weights_total"] += int(prm.p.size)
            out["weights_differ"] += nm
            out["weights_max_ulp"] = max(out["weights_max_ulp"], mu)
        for k in ("row", "col", "v", "max_v"):
            if f"s{i}_{k}" in gold:
                out["state_max_rel"] = max(out["state_max_rel"], rel_err(prm.state[k], gold[f"s{i}_{k}"]))
        for k in _MOM:
            if f"{k}_scale" in prm.state:
                out["scale_max_ulp"] = max(out["scale_max_ulp"],
                                           f32_ulps(prm.state[f"{k}_scale"], gold[f"s{i}_{k}_scale"]))
            if k in prm.state:
                a, b = prm.state[k].reshape(-1), gold[f"s{i}_{k}"].reshape(-1)
                out["codes_total"] += int(a.size)
                out["codes_differ"] += int((a != b).sum())
    return out


def f32_case(name: str) -> dict:
    case = CASES[name]
    gold = load_golden(name)
    params, _opt, evalp = run_oracle(case)
    out = {"kind": "f32", "weights_max_rel": 0.0, "state_max_rel": 0.0, "momentum_max_rel": 0.0,
           "weights_differ": 0, "weights_total": 0}
    for i, prm in enumerate(params):
        ref = gold[f"p{i}"]
        out["weights_max_rel"] = max(out["weights_max_rel"], rel_err(prm.p, ref))
        out["weights_differ"] += int((prm.p.reshape(-1) != ref.reshape(-1)).sum())
        out["weights_total"] += int(prm.p.size)
        if evalp is not None:
            out["weights_max_rel"] = max(out["weights_max_rel"], rel_err(evalp[i], gold[f"p{i}_eval"]))
        for k in ("row", "col", "v", "max_v"):
            if f"s{i}_{k}" in gold:
                out["state_max_rel"] = max(out["state_max_rel"], rel_err(prm.state[k], gold[f"s{i}_{k}"]))
        for k in _MOM:
            if k in prm.state and prm.state[k].dtype == np.float32:
                out["momentum_max_rel"] = max(out["momentum_max_rel"],
                                              rel_err(prm.state[k], gold[f"s{i}_{k}"].reshape(prm.state[k].shape)))
    return out


def cfg0_case() -> dict:
    gold = load_golden("cfg0")
    params, _opt, _ = run_oracle(CFG0)
    s = CFG0["sample_stride"]
    out = {"kind": "cfg0", "sample_total": 0, "sample_differ": 0, "sample_max_ulp": 0, "state_max_rel": 0.0,
           "per_param": []}
    for i, prm in enumerate(params):
        for k in ("row", "col"):
            out["state_max_rel"] = max(out["state_max_rel"], rel_err(prm.state[k], gold[f"s{i}_{k}"]))
        mine = prm.p.reshape(-1)[::s]
        nm, mu = bf16_mismatch(mine, gold[f"p{i}_sample"])
        out["sample_total"] += int(mine.size)
        out["sample_differ"] += nm
        out["sample_max_ulp"] = max(out["sample_max_ulp"], mu)
        out["per_param"].append({"shape": list(prm.shape), "sampled": int(mine.size), "differ": nm, "max_ulp": mu})
    return out


def pd_case(name: str) -> dict:
    case = CASES[name]
    gold = load_golden(name)
    params, opt = build_oracle(case)
    traj = []
    for step in range(1, case["steps"] + 1):
        set_grads(case, params, step)
        opt.step()
        traj.append(opt.group["d"])
    out = {"kind": "kprodigy", "d_max_rel": rel_err(np.array(traj), gold["d_traj"]), "weights_differ": 0,
           "weights_total": 0, "weights_max_rel": 0.0, "codes_differ_outside_tail": 0, "state_max_rel": 0.0}
    for i, prm in enumerate(params):
        if prm.p_dtype == O.BF16:
            nm, _ = bf16_mismatch(prm.p, gold[f"p{i}"])
            out["weights_differ"] += nm
        else:
            out["weights_max_rel"] = max(out["weights_max_rel"], rel_err(prm.p, gold[f"p{i}"]))
        out["weights_total"] += int(prm.p.size)
        for k in ("row", "col", "v"):
            if f"s{i}_{k}" in gold:
                out["state_max_rel"] = max(out["state_max_rel"], rel_err(prm.state[k], gold[f"s{i}_{k}"]))
        if "m" in prm.state and prm.state["m"].dtype != np.float32:
            a, b = prm.state["m"].reshape(-1), gold[f"s{i}_m"].reshape(-1)
            tail = prm.numel % 32 if case["kwargs"].get("momentum_dtype", "bfloat16") == "bfloat16" else 0
            head = a.size - tail
            out["codes_differ_outside_tail"] += int((a[:head] != b[:head]).sum())
    return out


def main() -> None:
    from test_oracle_golden import BIT_CASES, F32_CASES, PD_CASES

    budgets = {}
    for name in BIT_CASES:
        budgets[name] = bit_case(name)
    for name in F32_CASES:
        budgets[name] = f32_case(name)
    for name in PD_CASES:
        budgets[name] = pd_case(name)
    budgets["cfg0"] = cfg0_case()
    path = os.path.join(HERE, "oracle_budgets.json")
    with open(path, "w") as fh:
        json.dump(budgets, fh, indent=1, sort_keys=True)
        fh.write("\n")
    for k, v in sorted(budgets.items()):
        print(k, {kk: vv for kk, vv in v.items() if kk != "per_param"})


if __name__ == "__main__":
    main()
