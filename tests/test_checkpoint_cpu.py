"""Checkpoint interop with the reference layout (CPU: layout and loading only).

The golden fixtures hold the reference's own state after its steps
(tests/golden/make_golden.py ran kaon 0.7.4): per param the keys, dtypes and
shapes of ``optimizer.state`` (adakaon.py:318-335, lion.py:210-241,
adapnm.py:451-500, kprodigy.py:262-291, _momentum_codec.py:253-406).  These tests check that

* kaon_amd's fresh state has the reference's keys and dtypes, and its shapes
  except where the reference's own two paths differ (the 1-D int8 scales:
  ``()`` at init and on the foreach path, ``(1,)`` after the per-param requant,
  tests/test_fused_triton.py:906-908 of the reference);
* a reference-layout checkpoint loads with every tensor byte-identical, both
  shapes of the 1-D scale included, for bf16 and fp32 params;
* kaon_amd's own state_dict round-trips through torch.save / torch.load
  (weights_only) with its SR key.

Stepping from a loaded checkpoint runs in tests/test_gpu_checkpoint.py.
"""
import io

import numpy as np
import pytest
import torch

from cases import CASES, grad_values, param_values
from golden_compare import load_golden
from gpu_cases import make_opt

INTEROP = [k for k, c in CASES.items() if c["opt"] in ("adakaon", "lion", "adapnm", "kprodigy")]


def _tdt(name):
    return {"bf16": torch.bfloat16, "f16": torch.float16}.get(name, torch.float32)


def _cpu_opt(case):
    pdt = _tdt(case["p_dtype"])
    params = []
    for i, _ in enumerate(case["shapes"]):
        p = torch.nn.Parameter(torch.from_numpy(param_values(case, i)).to(pdt))
        p.grad = torch.from_numpy(grad_values(case, i, 1)).to(_tdt(case["g_dtype"]))
        params.append(p)
    opt = make_opt(case, params)
    for g in opt.param_groups:
        for p in g["params"]:
            opt._init_state(p, opt.state[p], g)
    return opt, params


def _golden_state(gold, i, p_dtype="bf16"):
    """The fixture's state of param i as torch tensors; 16-bit arrays are bf16
    momenta, or the kahan shift in the param dtype."""
    out = {}
    pre = f"s{i}_"
    for k, a in gold.items():
        if not k.startswith(pre):
            continue
        key = k[len(pre):]
        if key.endswith("_numel") or key.endswith("_block") or key == "step":  # ints
            out[key] = int(a)
        elif a.dtype == np.uint16:  # 16-bit float bits
            dt = _tdt(p_dtype) if key == "shift" else torch.bfloat16
            out[key] = torch.from_numpy(a.view(np.int16).copy()).view(dt)
        else:
            out[key] = torch.from_numpy(a.copy())
    return out


def _bytes(t):
    return t.detach().contiguous().reshape(-1).view(torch.uint8).numpy()


def _reference_sd(name, opt):
    gold = load_golden(name)
    sd = opt.state_dict()
    sd["state"] = {i: _golden_state(gold, i, CASES[name]["p_dtype"]) for i in range(len(CASES[name]["shapes"]))}
    sd.pop("kaon_amd", None)
    return sd, gold


@pytest.mark.parametrize("name", INTEROP)
def test_fresh_state_has_the_reference_layout(name):
    case = CASES[name]
    opt, params = _cpu_opt(case)
    gold = load_golden(name)
    for i, p in enumerate(params):
        ref = _golden_state(gold, i, case["p_dtype"])
        st = opt.state[p]
        assert sorted(st) == sorted(ref), (name, i, sorted(st), sorted(ref))
        for k, v in ref.items():
            if k == "step":  # KProdigy's per-param step count: an int, 0 when fresh
                assert isinstance(st[k], int) and st[k] == 0, (name, i, k)
                continue
            if not torch.is_tensor(v):
                assert int(st[k]) == v, (name, i, k)
                continue
            assert st[k].dtype == v.dtype, (name, i, k, st[k].dtype, v.dtype)
            if k.endswith("_scale") and p.ndim == 1 and v.dtype == torch.float32 and case["kwargs"].get(
                    "momentum_dtype") == "int8":
                assert tuple(st[k].shape) == () and tuple(v.shape) in ((), (1,)), (name, i, v.shape)
            else:
                assert st[k].shape == v.shape, (name, i, k, tuple(st[k].shape), tuple(v.shape))


@pytest.mark.parametrize("name", INTEROP)
def test_reference_checkpoint_loads_byte_identical(name):
    case = CASES[name]
    opt, params = _cpu_opt(case)
    sd, gold = _reference_sd(name, opt)
    opt.load_state_dict(sd)
    for i, p in enumerate(params):
        ref = _golden_state(gold, i, case["p_dtype"])
        st = opt.state[p]
        for k, v in ref.items():
            if not torch.is_tensor(v):
                assert int(st[k]) == v
                continue
            assert st[k].dtype == v.dtype and st[k].shape == v.shape, (name, i, k)
            assert np.array_equal(_bytes(st[k]), _bytes(v)), (name, i, k)


def test_bf16_params_keep_fp32_state_exact():
    """torch's load rounds floating state to the param dtype; the loader restores
    the saved fp32 row/col/v/scales rather than casting the rounded values back."""
    name = "ada_int8_sr"
    opt, params = _cpu_opt(CASES[name])
    assert params[0].dtype == torch.bfloat16
    sd, gold = _reference_sd(name, opt)
    opt.load_state_dict(sd)
    row = opt.state[params[0]]["row"]
    assert row.dtype == torch.float32
    assert np.array_equal(row.numpy(), gold["s0_row"])
    # the values are not all bf16-representable, so a lossy round trip would show
    assert not np.array_equal(gold["s0_row"], torch.from_numpy(gold["s0_row"]).bfloat16().float().numpy())


@pytest.mark.parametrize("name", ["ada_int8_sr", "ada_4bit_sr", "lion_bf16_sr"])
def test_state_dict_round_trip_through_torch_save(name):
    case = CASES[name]
    opt, params = _cpu_opt(case)
    sd0, _ = _reference_sd(name, opt)
    opt.load_state_dict(sd0)
    opt._t, opt.sr_seed = 7, 1234
    buf = io.BytesIO()
    torch.save(opt.state_dict(), buf)
    buf.seek(0)
    sd = torch.load(buf, weights_only=True)
    assert sd["kaon_amd"] == {"step": 7, "sr_seed": 1234}
    opt2, params2 = _cpu_opt(case)
    opt2.load_state_dict(sd)
    assert (opt2._t, opt2.sr_seed) == (7, 1234)
    for p, q in zip(params, params2):
        a, b = opt.state[p], opt2.state[q]
        assert sorted(a) == sorted(b)
        for k in a:
            if torch.is_tensor(a[k]):
                assert a[k].dtype == b[k].dtype and a[k].shape == b[k].shape
                assert np.array_equal(_bytes(a[k]), _bytes(b[k])), (name, k)
            else:
                assert a[k] == b[k]


def test_nekaon_load_clears_the_climb():
    """MSAM.load_state_dict (msam.py:409-421): checkpoints are saved in eval mode,
    so no climb is active after loading."""
    from kaon_amd import Nekaon

    p = torch.nn.Parameter(torch.zeros(8, 16, dtype=torch.bfloat16))
    opt = Nekaon([p], lr=1e-3)
    sd = opt.state_dict()
    opt._has_e, opt._eclamp = True, {0: 0.1}
    opt.load_state_dict(sd)
    assert opt._has_e is False and opt._eclamp == {}


def test_msam_load_clears_the_climb_and_validates():
    """MSAM.load_state_dict (msam.py:409-421) clears the climb and the cached norm;
    the constructor checks follow msam.py:101-108."""
    from kaon_amd import MSAM

    p = torch.nn.Parameter(torch.zeros(8, 16, dtype=torch.bfloat16))
    opt = MSAM([p], rho=0.3, lr=1e-3)
    sd = opt.state_dict()
    assert "msam" in sd
    opt._has_e, opt._mnorm, opt._eclamp = True, 0.5, {0: 0.1}
    opt.load_state_dict(sd)
    assert opt._has_e is False and opt._mnorm == 0.0 and opt._eclamp == {}
    with pytest.raises(ValueError):
        MSAM([p], norm="layer")
    with pytest.raises(ValueError):
        MSAM([p], eps=-1.0)
    assert MSAM([p], norm="tensor").norm == "tensor"


# ---------------------------------------------------------------- the other direction
# tests/golden/make_interop.py wrote kaon_amd checkpoints (the state_dict of a
# kaon_amd optimizer holding the oracle's state after the case's first steps),
# loaded each into the reference optimizer and let it take the last step.
INTEROP_BACK = ("ada_int8_sr", "ada_4bit_sr", "ada_bf16_rn", "ada_kahan", "lion_int8_sr", "lion_4bit_rn")


def _interop(name):
    import os

    here = os.path.dirname(os.path.abspath(__file__))
    return dict(np.load(os.path.join(here, "golden", f"interop_{name}.npz")))


@pytest.mark.parametrize("name", INTEROP_BACK)
def test_reference_resumes_from_a_kaon_amd_checkpoint(name):
    """The oracle, restarted from the checkpoint the reference loaded, takes the
    same last step in torch CPU's reduction order: identical weights, codes,
    scales and fp32 state to what the reference wrote.  For bf16 params the
    reference's own loader rounds the fp32 state (row, col, v, scales) to bf16
    on the way in, for its own checkpoints as for these; the restart does the same."""
    import oracle as O
    from golden_compare import build_oracle, set_grads

    case = CASES[name]
    fx = _interop(name)
    assert int(fx["c_step"]) == case["steps"] - 1
    oparams, oopt = build_oracle(case)
    for i, prm in enumerate(oparams):
        prm.p[...] = fx[f"cp{i}"].reshape(prm.p.shape)
        for k in list(prm.state):
            key = f"c{i}_{k}"
            if k.startswith("_") or key not in fx:
                continue
            v = fx[key]
            if np.ndim(prm.state[k]) == 0 and not isinstance(prm.state[k], np.ndarray):
                prm.state[k] = type(prm.state[k])(v)
                continue
            v = v.reshape(np.shape(prm.state[k])).astype(np.asarray(prm.state[k]).dtype)
            if case["p_dtype"] == "bf16" and v.dtype == np.float32:
                # the reference's load: torch's Optimizer.load_state_dict casts floating
                # state to the param dtype, and load_state_dict_preserving_dtypes
                # (_momentum_codec.py:417-452) casts the rounded values back to fp32
                v = O.bf16_to_f32(O.f32_to_bf16(v)).reshape(v.shape)
            prm.state[k] = v
    set_grads(case, oparams, case["steps"])
    oopt.t = case["steps"] - 1  # the SR noise of the last step is keyed on its step number
    with O.torch_order():
        oopt.step()
    for i, prm in enumerate(oparams):
        assert np.array_equal(prm.p.reshape(-1), fx[f"p{i}"].reshape(-1)), (name, i, "weights")
        for k, v in prm.state.items():
            key = f"s{i}_{k}"
            if k.startswith("_") or key not in fx:
                continue
            a = np.asarray(v).reshape(-1)
            b = fx[key].reshape(-1)
            if a.dtype != b.dtype and a.itemsize == b.itemsize:
                b = b.view(a.dtype)
            assert np.array_equal(a, b.astype(a.dtype)), (name, i, k)
