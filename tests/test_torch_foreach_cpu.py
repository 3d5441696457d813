"""Pin oracle/torch_foreach.py, the torch-CPU restatement of the reference's native
foreach step that bench.py times as the CPU baseline, against the reference's own
output (the golden fixtures, written by kaon 0.7.4 on torch CPU with the library's
Philox noise injected into its stochastic rounding).

Each case steps the restatement on the case's inputs with the same routing the
fixture used (``foreach`` from the case: RN / fp32 cases ran the stacked buckets,
SR cases the per-param path) and the same noise, and must give the reference's
weights, momentum and factored state bit for bit.  A second check runs every
case through the stacked buckets and the per-param path and requires the same
bits, as the reference's own foreach-vs-per-param tests do.
"""
import numpy as np
import pytest
import torch

import oracle as O
import torch_foreach as TF
from cases import grad_values, param_values
from golden_compare import CASES, group_for, load_golden

torch.set_num_threads(1)

NAMES = sorted(k for k, c in CASES.items() if c["opt"] in ("adakaon", "lion")
               and c["kwargs"].get("momentum_dtype", "bfloat16") != "4bit")


def _tdt(name):
    return {"bf16": torch.bfloat16, "f16": torch.float16}.get(name, torch.float32)


def _run(case, foreach=None):
    g = group_for(case)
    ps = [torch.from_numpy(param_values(case, i)).to(_tdt(case["p_dtype"])) for i in range(len(case["shapes"]))]
    gs = [torch.zeros(1)] * len(ps)
    cls = TF.ForeachAdakaon if case["opt"] == "adakaon" else TF.ForeachLion
    fe = case["kwargs"].get("foreach", True) if foreach is None else foreach
    opt = cls(ps, gs, g, foreach=fe)
    ctx = {"step": 0}

    def noise(lo, hi, size, dtype):
        parts = [O.sr_noise(ps[i].numel(), case["seed"], ctx["step"], i, 1) for i in opt.writing]
        return torch.from_numpy(np.concatenate(parts).astype(np.int32)).reshape(size)

    opt.randint = noise
    for step in range(1, case["steps"] + 1):
        ctx["step"] = step
        opt.gs[:] = [torch.from_numpy(grad_values(case, i, step)).to(_tdt(case["g_dtype"]))
                     for i in range(len(ps))]
        opt.step()
    return ps, opt


def _bits(t):
    t = t.contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


@pytest.mark.parametrize("name", NAMES)
def test_restatement_reproduces_the_reference(name):
    case = CASES[name]
    gold = load_golden(name)
    ps, opt = _run(case)
    for i, p in enumerate(ps):
        assert np.array_equal(_bits(p).reshape(-1), gold[f"p{i}"].reshape(-1)), (name, i)
        st = opt.state[i]
        for k in ("row", "col", "v", "m", "m_scale"):
            if k in st and f"s{i}_{k}" in gold:
                a, b = _bits(st[k]).reshape(-1), gold[f"s{i}_{k}"].reshape(-1)
                if a.dtype != b.dtype and a.itemsize == b.itemsize:
                    a = a.view(b.dtype)
                assert np.array_equal(a, b), (name, i, k)


@pytest.mark.parametrize("name", ["ada_int8_sr", "ada_bf16_rn", "lion_int8_sr", "lion_bf16_sr"])
def test_stacked_buckets_equal_the_per_param_path(name):
    case = dict(CASES[name])
    case["shapes"] = [[8, 16], [8, 16], [16, 8, 3, 3], [16, 8, 3, 3], [40], [40]]
    a, _ = _run(case, foreach=True)
    b, _ = _run(case, foreach=False)
    for x, y in zip(a, b):
        assert np.array_equal(_bits(x), _bits(y)), name


def test_routing_follows_the_budget():
    """CPU stack budget min(64M, 4 * cutoff); per-param above min(cutoff, budget // 2)."""
    assert TF.cpu_stack_budget() == 8_000_000
    assert TF.cpu_stack_budget(100) == 400
    ps = [torch.zeros(10, 10), torch.zeros(10, 10), torch.zeros(3000)]
    opt = TF.ForeachAdakaon(ps, [torch.zeros_like(p) for p in ps], group_for(CASES["ada_bf16_rn"]), cutoff=1000)
    fast, slow = opt._route(True)
    assert fast == [0, 1] and slow == [2]
