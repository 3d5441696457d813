"""Resuming from checkpoints on the GPU, bit for bit.

* From a reference checkpoint: the golden fixtures hold kaon 0.7.4's params
  and state after its steps (tests/golden/make_golden.py).  They are loaded
  in the reference's layout into the HIP optimizer and, separately, into the
  CPU oracle; one more step with the case's next gradients must give identical
  weights, codes, scales and fp32 state on both.  The reference keys its SR
  noise on the global torch RNG, so a loaded checkpoint carries no SR key; both
  sides continue from step count 0 with the case's seed.
* From kaon_amd's own checkpoint: 3 steps, torch.save / torch.load
  (weights_only) into a fresh optimizer over copies of the params, 2 more
  steps; identical to 5 uninterrupted steps (the SR key is restored).
"""
import io

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

import oracle as O  # noqa: E402
from cases import CASES, grad_values  # noqa: E402
from golden_compare import group_for, load_golden  # noqa: E402
from gpu_cases import DEV, assert_same_as_oracle, make_opt, run_gpu, state_of, to_bits, tdtype  # noqa: E402

RESUME = [k for k, c in CASES.items() if c["opt"] in ("adakaon", "lion")]


@pytest.fixture(autouse=True, scope="module")
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")


def _golden_state(gold, i):
    out = {}
    pre = f"s{i}_"
    for k, a in gold.items():
        if k.startswith(pre):
            out[k[len(pre):]] = a
    return out


def _torch_state(st, pdt=torch.bfloat16):
    """16-bit arrays are bf16 momenta, or the kahan shift in the param dtype."""
    out = {}
    for k, a in st.items():
        if k in ("m_numel", "m_block"):
            out[k] = int(a)
        elif a.dtype == np.uint16:
            out[k] = torch.from_numpy(a.view(np.int16).copy()).view(pdt if k == "shift" else torch.bfloat16)
        else:
            out[k] = torch.from_numpy(a.copy())
    return out


def _param_tensor(a, pdt):
    if pdt in (torch.bfloat16, torch.float16):
        return torch.from_numpy(a.view(np.int16).copy()).view(pdt).to(DEV)
    return torch.from_numpy(a.astype(np.float32)).to(DEV)


@pytest.mark.parametrize("name", RESUME)
def test_resume_from_reference_checkpoint(name):
    case = CASES[name]
    print(f"[gpu] resume from reference checkpoint {name}", flush=True)
    gold = load_golden(name)
    pdt, gdt = tdtype(case["p_dtype"]), tdtype(case["g_dtype"])
    nxt = case["steps"] + 1
    # HIP optimizer over the reference's params, reference state loaded
    params = [torch.nn.Parameter(_param_tensor(gold[f"p{i}"], pdt)) for i in range(len(case["shapes"]))]
    opt = make_opt(case, params)
    sd = opt.state_dict()
    sd.pop("kaon_amd", None)
    sd["state"] = {i: _torch_state(_golden_state(gold, i), pdt) for i in range(len(params))}
    opt.load_state_dict(sd)
    for i, p in enumerate(params):
        p.grad = torch.from_numpy(grad_values(case, i, nxt)).to(DEV, gdt)
    opt.step()
    torch.cuda.synchronize()
    # oracle from the same params and state
    dt = {"bf16": O.BF16, "f16": O.F16}.get(case["p_dtype"], O.F32)
    gt = {"bf16": O.BF16, "f16": O.F16}.get(case["g_dtype"], O.F32)
    oparams = []
    for i, shape in enumerate(case["shapes"]):
        pv = O.values(gold[f"p{i}"], dt)
        oparams.append(O.make_param(shape, dt, gt, tensor_id=i, p_values=pv))
    oopt = O.OracleOptimizer(oparams, case["opt"], group_for(case), seed=case["seed"])
    for i, prm in enumerate(oparams):
        for k, a in _golden_state(gold, i).items():
            if k in ("m_numel", "m_block"):
                prm.state[k] = int(a)
            else:
                prm.state[k] = np.ascontiguousarray(a).reshape(np.shape(prm.state[k])).copy()
        g = grad_values(case, i, nxt)
        if gt == O.BF16:
            prm.g = O.f32_to_bf16(g).reshape(prm.shape)
        elif gt == O.F16:
            prm.g = O.f32_to_f16(g).reshape(prm.shape)
        else:
            prm.g = g.copy()
    oopt.step()
    assert_same_as_oracle(case, oparams, params, opt, label=f"resume {name}")
    # the loaded 1-D int8 scale keeps the checkpoint's shape through the step
    for i, p in enumerate(params):
        ms = _golden_state(gold, i).get("m_scale")
        if ms is not None:
            assert tuple(state_of(opt, p)["m_scale"].shape) == ms.shape


@pytest.mark.parametrize("name", ["ada_int8_sr", "ada_4bit_sr", "lion_bf16_sr", "ada_kahan"])
def test_save_load_resume_matches_uninterrupted(name):
    case = dict(CASES[name])
    print(f"[gpu] save/load resume {name}", flush=True)
    full = dict(case, steps=5)
    ref_params, ref_opt, _ = run_gpu(full)
    part = dict(case, steps=3)
    params, opt, _ = run_gpu(part)
    buf = io.BytesIO()
    torch.save(opt.state_dict(), buf)
    buf.seek(0)
    sd = torch.load(buf, weights_only=True)
    gdt = tdtype(case["g_dtype"])
    params2 = [torch.nn.Parameter(p.detach().clone()) for p in params]
    opt2 = make_opt(case, params2)
    opt2.load_state_dict(sd)
    for step in (4, 5):
        for i, p in enumerate(params2):
            p.grad = torch.from_numpy(grad_values(case, i, step)).to(DEV, gdt)
        opt2.step()
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(ref_params, params2)):
        assert np.array_equal(to_bits(a), to_bits(b)), (name, i, "weights")
        sa, sb = state_of(ref_opt, a), state_of(opt2, b)
        for k in sa:
            if torch.is_tensor(sa[k]):
                assert np.array_equal(to_bits(sa[k]).reshape(-1), to_bits(sb[k]).reshape(-1)), (name, i, k)
            else:
                assert sa[k] == sb[k], (name, i, k)


INTEROP_BACK = ("ada_int8_sr", "ada_4bit_sr", "ada_bf16_rn", "ada_kahan", "lion_int8_sr", "lion_4bit_rn")


@pytest.mark.parametrize("name", INTEROP_BACK)
def test_state_dict_is_the_checkpoint_the_reference_resumed_from(name):
    """tests/golden/make_interop.py loaded a kaon_amd checkpoint into the reference
    and let it step (tests/test_checkpoint_cpu.py replays that step).  The HIP
    optimizer's own state_dict after the same first steps is that checkpoint:
    the same keys, dtypes, shapes and bytes for the weights and every state
    tensor, and the same step count and SR key."""
    import os

    here = os.path.dirname(os.path.abspath(__file__))
    fx = dict(np.load(os.path.join(here, "golden", f"interop_{name}.npz")))
    case = dict(CASES[name], steps=CASES[name]["steps"] - 1)
    print(f"[gpu] state_dict vs interop checkpoint {name}", flush=True)
    params, opt, _ = run_gpu(case)
    buf = io.BytesIO()
    torch.save(opt.state_dict(), buf)
    buf.seek(0)
    sd = torch.load(buf, weights_only=True)
    assert int(sd["kaon_amd"]["step"]) == int(fx["c_step"])
    assert int(sd["kaon_amd"]["sr_seed"]) == int(fx["c_sr_seed"])
    for i, p in enumerate(params):
        assert np.array_equal(to_bits(p), fx[f"cp{i}"]), (name, i, "weights")
        want = {k[len(f"c{i}_"):] for k in fx if k.startswith(f"c{i}_")}
        assert sorted(sd["state"][i]) == sorted(want), (name, i, sorted(sd["state"][i]), sorted(want))
        for k, v in sd["state"][i].items():
            ref = fx[f"c{i}_{k}"]
            if not torch.is_tensor(v):
                assert int(v) == int(ref), (name, i, k)
                continue
            got = to_bits(v)
            assert got.dtype == ref.dtype and got.shape == ref.shape, (name, i, k, got.dtype, got.shape, ref.shape)
            assert np.array_equal(got, ref), (name, i, k)
