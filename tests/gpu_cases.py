"""Run a golden case through the HIP optimizers on cuda:0 (helper for the gpu tests).

The case definitions and input generators are tests/golden/cases.py, shared
with the oracle replay in tests/golden_compare.py, so both sides step on the
same bytes.  The SR key matches the oracle's (seed = case seed, step count,
param index, stream), so stochastic rounding is compared bit for bit.
"""
from __future__ import annotations

import numpy as np
import torch

import oracle as O
from cases import grad_values, param_values
from golden_compare import group_for

DEV = torch.device("cuda:0")


def tdtype(name: str) -> torch.dtype:
    return {"bf16": torch.bfloat16, "f16": torch.float16}.get(name, torch.float32)


def make_opt(case, params, group=None, extra=None):
    """The kaon_amd optimizer of a case; ``extra`` adds constructor keywords (e.g.
    reduction_order="torch")."""
    from kaon_amd import MSAM, AdaMuon, AdaPNM, Adakaon, KProdigy, Lion, Nekaon

    g = dict(group or group_for(case))
    name = case["opt"]
    common = dict(momentum_dtype=g["momentum_dtype"], momentum_4bit_block=g["momentum_4bit_block"],
                  cautious=g["cautious"], gradient_centralization=g["gradient_centralization"],
                  bf16_method=g["bf16_method"])
    common.update(extra or {})
    if name == "adakaon":
        opt = Adakaon(params, lr=g["lr"], betas=g["betas"], eps=g["eps"], weight_decay=g["weight_decay"],
                      clip_threshold=g["clip_threshold"], **common)
        opt.sr_seed = case["seed"]
    elif name == "lion":
        opt = Lion(params, lr=g["lr"], betas=g["betas"], weight_decay=g["weight_decay"], **common)
        opt.sr_seed = case["seed"]
    elif name == "nekaon":
        md = common.pop("momentum_dtype")
        opt = Nekaon(params, lr=g["lr"], k=g["k"], betas=g["betas"], weight_decay=g["weight_decay"],
                     momentum_dtype=md, eps=g["eps"], clip_threshold=g["clip_threshold"], **common)
        opt.inner.sr_seed = case["seed"]
    elif name == "msam":
        # MSAM takes ``eps`` for itself; the Adakaon base keeps its default eps
        opt = MSAM(params, rho=g["rho"], norm=g["norm"], eps=g["msam_eps"], lr=g["lr"], betas=g["betas"],
                   weight_decay=g["weight_decay"], clip_threshold=g["clip_threshold"], **common)
        opt.inner.sr_seed = case["seed"]
    elif name == "adamuon":
        opt = AdaMuon(params, lr=g["lr"], betas=g["betas"], eps=g["eps"], weight_decay=g["weight_decay"],
                      ns_steps=g["ns_steps"], clip_threshold=g["clip_threshold"], **common)
        opt.sr_seed = case["seed"]
    elif name == "kprodigy":
        kw = {k: g[k] for k in ("lr", "betas", "beta3", "eps", "weight_decay", "decouple", "use_bias_correction",
                                "safeguard_warmup", "d0", "d_coef", "growth_rate", "d_update_freq", "slice_p",
                                "momentum_dtype", "momentum_4bit_block", "second_moment", "eps_factored", "cautious",
                                "gradient_centralization", "bf16_method", "factor_conv_as_matrix")}
        opt = KProdigy(params, **kw)
        opt.sr_seed = case["seed"]
    elif name == "adapnm":
        opt = AdaPNM(params, lr=g["lr"], betas=g["betas"], beta0=g["beta0"], eps=g["eps"],
                     weight_decay=g["weight_decay"], clip_threshold=g["clip_threshold"], ams_bound=g["ams_bound"],
                     **common)
        opt.sr_seed = case["seed"]
    else:
        raise ValueError(name)
    return opt


def to_bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().contiguous().cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    return t.numpy().copy()


def run_gpu(case, group=None, values=None, extra=None):
    """Step the HIP optimizer on the case; returns (params, opt, eval-mode weights or None)."""
    pdt, gdt = tdtype(case["p_dtype"]), tdtype(case["g_dtype"])
    params = []
    for i, _shape in enumerate(case["shapes"]):
        v = param_values(case, i) if values is None else values[i]
        prm = torch.nn.Parameter(torch.from_numpy(np.ascontiguousarray(v)).to(DEV, pdt))
        if gdt != pdt:
            prm.grad_dtype = gdt   # torch >= 2.9 checks grad dtype against this attribute
        params.append(prm)
    opt = make_opt(case, params, group, extra)
    for step in range(1, case["steps"] + 1):
        idle = case.get("no_grad", {}).get(step, ())
        for i, p in enumerate(params):
            if i in idle:  # no gradient for this param this step
                p.grad = None
                continue
            g = grad_values(case, i, step)
            p.grad = torch.from_numpy(g).to(DEV, gdt)
        opt.step()
    evalp = None
    if case.get("eval_train"):
        opt.eval()
        evalp = [to_bits(p) for p in params]
        opt.train()
    torch.cuda.synchronize()
    return params, opt, evalp


def state_of(opt, p):
    inner = getattr(opt, "inner", opt)
    return inner.state[p]


def assert_same_as_oracle(case, oparams, params, opt, evalp=None, oeval=None, label=""):
    """Bit-exact comparison of weights and every state tensor."""
    for i, (op, p) in enumerate(zip(oparams, params)):
        got = to_bits(p).reshape(-1)
        want = op.p.reshape(-1)
        nbad = int((got != want).sum())
        assert nbad == 0, f"{label} param {i} {tuple(p.shape)}: {nbad}/{got.size} weights differ"
        st = state_of(opt, p)
        for k, ov in op.state.items():
            if k.startswith("_"):  # the oracle's own scratch
                continue
            if k.endswith("_numel") or k.endswith("_block") or k == "step":  # ints
                assert int(st[k]) == int(ov), (label, i, k)
                continue
            gv = to_bits(st[k]).reshape(-1)
            ov = np.asarray(ov).reshape(-1)
            if gv.dtype != ov.dtype:
                gv = gv.view(ov.dtype) if gv.itemsize == ov.itemsize else gv.astype(ov.dtype)
            nbad = int((gv != ov).sum())
            assert nbad == 0, f"{label} param {i} state {k}: {nbad}/{gv.size} differ"
        if evalp is not None:
            nbad = int((evalp[i].reshape(-1) != oeval[i].reshape(-1)).sum())
            assert nbad == 0, f"{label} param {i} eval weights: {nbad} differ"


def oracle_case_run(case, group=None, values=None):
    from golden_compare import dt

    g = dict(group or group_for(case))
    params = []
    for i, shape in enumerate(case["shapes"]):
        v = param_values(case, i) if values is None else values[i]
        params.append(O.make_param(shape, dt(case["p_dtype"]), dt(case["g_dtype"]), tensor_id=i, p_values=v))
    opt = O.OracleOptimizer(params, case["opt"], g, seed=case["seed"])
    for step in range(1, case["steps"] + 1):
        idle = case.get("no_grad", {}).get(step, ())
        for i, prm in enumerate(params):
            if i in idle:
                prm.g = None
                continue
            gv = grad_values(case, i, step)
            if prm.g_dtype == O.BF16:
                prm.g = O.f32_to_bf16(gv).reshape(prm.shape)
            elif prm.g_dtype == O.F16:
                prm.g = O.f32_to_f16(gv).reshape(prm.shape)
            else:
                prm.g = gv.copy()
        opt.step()
    evalp = None
    if case.get("eval_train"):
        opt.msam_apply(-1.0)
        evalp = [prm.p.copy() for prm in params]
        opt.msam_apply(+1.0)
    return params, opt, evalp
