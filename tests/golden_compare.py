"""Helpers that replay a golden case through the oracle and compare.

Used by tests/test_oracle_golden.py (CPU) and by the GPU parity tests.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
sys.path.insert(0, os.path.join(os.path.dirname(HERE), "oracle"))

import oracle as O  # noqa: E402
from cases import CASES, CFG0, grad_values, param_values  # noqa: E402

# Constructor defaults of each reference optimizer (what the case kwargs do not set):
# Adakaon src/kaon/adakaon.py:195-218, Lion src/kaon/lion.py:152-171,
# AdaMuon src/kaon/adamuon.py:216-239, Nekaon src/kaon/nekaon.py:122-137, MSAM src/kaon/msam.py:101-108
# over Adakaon's (its eps is msam_eps here: Adakaon has an eps of its own),
# AdaPNM src/kaon/adapnm.py:344-370, KProdigy src/kaon/kprodigy.py:155-235 (the group keys d, d_max,
# d_numerator, k are its per-group D state).
DEFAULTS = {
    "adakaon": dict(lr=1e-3, betas=(0.9, 0.999), eps=(1e-30, 1e-3), weight_decay=0.0, clip_threshold=1.0,
                    momentum_dtype="bfloat16", momentum_4bit_block=128, cautious=True,
                    gradient_centralization=True, bf16_method="stochastic_rounding"),
    "lion": dict(lr=1e-4, betas=(0.9, 0.99), weight_decay=0.0, momentum_dtype="bfloat16",
                 momentum_4bit_block=128, cautious=True, gradient_centralization=True,
                 bf16_method="stochastic_rounding"),
    "adamuon": dict(lr=2e-2, betas=(0.95, 0.999), eps=(1e-30, 1e-3), weight_decay=0.0, ns_steps=2,
                    clip_threshold=1.0, momentum_dtype="bfloat16", momentum_4bit_block=128, cautious=True,
                    gradient_centralization=False, bf16_method="stochastic_rounding"),
    "nekaon": dict(lr=1e-3, k=1.5, betas=(0.5, 0.999), eps=(1e-30, 1e-3), weight_decay=0.1,
                   clip_threshold=1.0, momentum_dtype="4bit", momentum_4bit_block=128, cautious=True,
                   gradient_centralization=True, bf16_method="stochastic_rounding"),
    "msam": dict(lr=1e-3, betas=(0.9, 0.999), eps=(1e-30, 1e-3), weight_decay=0.0, clip_threshold=1.0,
                 momentum_dtype="bfloat16", momentum_4bit_block=128, cautious=True,
                 gradient_centralization=True, bf16_method="stochastic_rounding", rho=0.3, norm="global",
                 msam_eps=1e-12),
    "kprodigy": dict(lr=1.0, betas=(0.9, 0.999), beta3=None, eps=1e-8, weight_decay=0.0, decouple=True,
                     use_bias_correction=False, safeguard_warmup=False, d=1e-6, d0=1e-6, d_max=1e-6,
                     d_numerator=0.0, d_coef=1.0, growth_rate=float("inf"), d_update_freq=1, slice_p=1, k=0,
                     momentum_dtype="bfloat16", momentum_4bit_block=128, second_moment="full",
                     eps_factored=1e-30, cautious=False, gradient_centralization=True,
                     bf16_method="stochastic_rounding", factor_conv_as_matrix=True),
    "adapnm": dict(lr=1e-3, betas=(0.8, 0.999), beta0=0.5, eps=1e-8, weight_decay=0.0, clip_threshold=1.0,
                   cautious=True, gradient_centralization=True, ams_bound=False, momentum_dtype="bfloat16",
                   momentum_4bit_block=128, bf16_method="stochastic_rounding"),
}
_IGNORED = ("foreach", "foreach_batch_cutoff", "foreach_stack_budget", "fused")


def group_for(case) -> dict:
    g = dict(DEFAULTS[case["opt"]])
    for k, v in case["kwargs"].items():
        if k not in _IGNORED:
            g[k] = v
    if case["opt"] == "kprodigy" and "d0" in case["kwargs"]:
        g["d"] = g["d_max"] = case["kwargs"]["d0"]
    return g


def dt(name: str) -> int:
    return {"bf16": O.BF16, "f16": O.F16}.get(name, O.F32)


def build_oracle(case):
    params = []
    for i, shape in enumerate(case["shapes"]):
        params.append(O.make_param(shape, dt(case["p_dtype"]), dt(case["g_dtype"]), tensor_id=i,
                                   p_values=param_values(case, i)))
    opt = O.OracleOptimizer(params, case["opt"], group_for(case), seed=case["seed"])
    return params, opt


def set_grads(case, params, step):
    for i, prm in enumerate(params):
        g = grad_values(case, i, step)
        if prm.g_dtype == O.BF16:
            prm.g = O.f32_to_bf16(g).reshape(prm.shape)
        elif prm.g_dtype == O.F16:
            prm.g = O.f32_to_f16(g).reshape(prm.shape)
        else:
            prm.g = g.copy()


def run_oracle(case):
    params, opt = build_oracle(case)
    for step in range(1, case["steps"] + 1):
        set_grads(case, params, step)
        opt.step()
    evalp = None
    if case.get("eval_train"):
        opt.msam_apply(-1.0)
        evalp = [prm.p.copy() for prm in params]
        opt.msam_apply(+1.0)
    return params, opt, evalp


def load_golden(name):
    return dict(np.load(os.path.join(HERE, "golden", f"{name}.npz")))


def bf16_mismatch(a_bits: np.ndarray, b_bits: np.ndarray) -> tuple[int, int]:
    """(#elements differing, max difference in bf16 ulps) between two bf16 bit arrays."""
    a = a_bits.astype(np.int32).reshape(-1)
    b = b_bits.astype(np.int32).reshape(-1)
    # map sign-magnitude to a monotone integer line
    a = np.where(a & 0x8000, -(a & 0x7FFF), a)
    b = np.where(b & 0x8000, -(b & 0x7FFF), b)
    d = np.abs(a - b)
    return int((d != 0).sum()), int(d.max()) if d.size else 0


def rel_err(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, dtype=np.float64).reshape(-1)
    b = np.asarray(b, dtype=np.float64).reshape(-1)
    den = np.maximum(np.abs(b), 1e-30)
    return float(np.max(np.abs(a - b) / den)) if a.size else 0.0


__all__ = ["CASES", "CFG0", "DEFAULTS", "bf16_mismatch", "build_oracle", "group_for", "load_golden",
           "rel_err", "run_oracle", "set_grads"]
