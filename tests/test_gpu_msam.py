"""MSAM on the GPU against the oracle, bit for bit.

The oracle's MSAM (oracle/oracle.py OracleOptimizer "msam") matches the
reference's own output on the golden cases (tests/test_oracle_golden.py: with
the reference's norms fed in, the weights are bit-exact, and the norm of the
reference's momentum is within 4 fp32 ulps of the reference's).  Here
kaon_amd.MSAM must reproduce the oracle exactly: weights, momentum codes and
scales, factored state, eval-mode weights, and the norm itself -- the GPU's
per-tensor sums of squares (kaon_momentum_sumsq) follow the oracle's 64-lane
order and are added on the host in the same param order, so ||m|| agrees to
the bit.  Over Adakaon the removal rides inside the Adakaon apply pass; over
another optimizer (Lion here) every perturbation is its own kaon_msam_apply
pass, checked against the oracle driven the same way by hand.
"""
import ctypes
import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

import oracle as O  # noqa: E402
from cases import grad_values, param_values  # noqa: E402
from golden_compare import CASES, group_for  # noqa: E402
from gpu_cases import DEV, assert_same_as_oracle, oracle_case_run, run_gpu, to_bits  # noqa: E402

GOLDEN = [k for k, c in CASES.items() if c["opt"] == "msam"]


@pytest.fixture(autouse=True, scope="module")
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")


def _check(case, label):
    oparams, oopt, oeval = oracle_case_run(case)
    params, opt, evalp = run_gpu(case)
    assert_same_as_oracle(case, oparams, params, opt, evalp=evalp, oeval=oeval, label=label)
    g = group_for(case)
    if g["norm"] == "global":
        assert opt._mnorm == oopt.mnorm, (label, opt._mnorm, oopt.mnorm)
        assert (opt._mnorm > 0.0) == (g["rho"] != 0.0)


@pytest.mark.parametrize("name", GOLDEN)
def test_golden_case_bit_exact(name):
    print(f"[gpu] msam golden {name}", flush=True)
    _check(CASES[name], name)


def _case(shapes, kwargs, steps=4, p="bf16", g="bf16", seed=5):
    return dict(steps=steps, seed=seed, p_dtype=p, g_dtype=g, opt="msam", shapes=shapes, kwargs=kwargs,
                eval_train=True)


EXTRA = {
    # several runs per tensor, long 1-D rows, int8 / 4-bit / bf16 / fp32 momentum
    "runs_int8": _case([[640, 64], [300, 72], [5120]], dict(lr=1e-3, rho=0.3, momentum_dtype="int8")),
    "runs_4bit": _case([[160, 40], [96, 24, 3, 3], [1000]], dict(lr=1e-3, rho=0.1, momentum_dtype="4bit",
                                                                 momentum_4bit_block=64)),
    "ragged_bf16": _case([[37, 45], [13, 7, 3], [101], [5, 3]], dict(lr=2e-3, rho=-0.3,
                                                                     momentum_dtype="bfloat16")),
    "f32_mom_f32p": _case([[48, 40], [64]], dict(lr=1e-3, rho=0.2, momentum_dtype="float32",
                                                  weight_decay=0.1), p="f32", g="f32"),
    "kahan_int8": _case([[40, 24], [56]], dict(lr=1e-3, rho=0.3, momentum_dtype="int8", bf16_method="kahan")),
    "none_4bit": _case([[160, 40], [33], [7, 9]], dict(lr=1e-3, rho=0.8, norm="none", momentum_dtype="4bit",
                                                       momentum_4bit_block=16)),
    "rho_zero": _case([[24, 32], [40]], dict(lr=1e-3, rho=0.0, momentum_dtype="int8")),
    # rows the specialized apply kernel takes (bf16 p and g, SR, GC, cautious): the removal
    # alone in its phase 6, and under weight decay in its phase 5 too
    "fast_bf16": _case([[320, 1280], [640, 640], [1280]], dict(lr=1e-3, rho=0.3, momentum_dtype="bfloat16")),
    "fast_int8_wd": _case([[320, 1280], [96, 64, 3, 3], [640]], dict(lr=1e-3, rho=-0.5, momentum_dtype="int8",
                                                                     weight_decay=0.1)),
    "fast_4bit_wd": _case([[256, 2048], [1280]], dict(lr=1e-3, rho=0.2, momentum_dtype="4bit", weight_decay=0.05)),
    # params with a momentum but no gradient on some steps: not stepped, but their climb
    # is removed and added again (msam.py:384-403); on step 3 of the Nekaon-form case no
    # param of the group has a gradient
    "gradless_global_int8": dict(_case([[320, 1280], [96, 64, 3, 3], [640], [24, 32]],
                                       dict(lr=1e-3, rho=0.3, momentum_dtype="int8")),
                                 no_grad={2: (1,), 3: (0, 2)}),
    "gradless_none_4bit": dict(_case([[160, 40], [33], [7, 9], [256, 64]],
                                     dict(lr=1e-3, rho=0.8, norm="none", momentum_dtype="4bit",
                                          momentum_4bit_block=16)),
                               no_grad={2: (0, 3), 3: (0, 1, 2, 3)}),
}


@pytest.mark.parametrize("name", sorted(EXTRA))
def test_extra_case_bit_exact(name):
    print(f"[gpu] msam extra {name}", flush=True)
    _check(EXTRA[name], name)


def test_rho_zero_is_plain_adakaon():
    """rho = 0 disables MSAM (msam.py:92-93): the weights are Adakaon's."""
    from kaon_amd import MSAM, Adakaon

    print("[gpu] msam rho=0 vs Adakaon", flush=True)
    torch.manual_seed(0)
    p0 = torch.randn(64, 48, device=DEV).bfloat16()
    a = torch.nn.Parameter(p0.clone())
    b = torch.nn.Parameter(p0.clone())
    oa = MSAM([a], rho=0.0, lr=1e-3, momentum_dtype="int8")
    ob = Adakaon([b], lr=1e-3, momentum_dtype="int8")
    oa.inner.sr_seed = ob.sr_seed = 3
    for s in range(3):
        g = torch.randn(64, 48, device=DEV).bfloat16() * 1e-2
        a.grad, b.grad = g.clone(), g.clone()
        oa.step()
        ob.step()
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_global_over_lion_base():
    """MSAM(base_optimizer=Lion): removal, Lion step, norm, climb as separate passes
    (msam.py:384-403), against the oracle's Lion driven the same way."""
    from kaon_amd import MSAM, Lion

    print("[gpu] msam global over Lion", flush=True)
    shapes = [[40, 24], [300, 72], [33]]
    case = dict(steps=4, seed=9, p_dtype="bf16", g_dtype="bf16", opt="lion", shapes=shapes,
                kwargs=dict(lr=1e-4, betas=(0.9, 0.99), momentum_dtype="int8", weight_decay=0.1))
    rho = 0.25
    g = group_for(case)
    # oracle, by hand
    oparams = [O.make_param(s, O.BF16, O.BF16, tensor_id=i, p_values=param_values(case, i))
               for i, s in enumerate(shapes)]
    oo = O.OracleOptimizer(oparams, "lion", g, seed=case["seed"])
    oo.rho, oo.norm, oo.meps = rho, "global", 1e-12
    has_e = False
    for step in range(1, case["steps"] + 1):
        for i, prm in enumerate(oparams):
            prm.g = O.f32_to_bf16(grad_values(case, i, step)).reshape(prm.shape)
        if has_e:
            oo.msam_apply(-1.0, step=step)
        oo.step()
        oo.mnorm = oo.global_mnorm()
        oo.msam_apply(+1.0)
        has_e = True
    oo.msam_apply(-1.0)
    oeval = [prm.p.copy() for prm in oparams]
    oo.msam_apply(+1.0)
    # GPU
    params = [torch.nn.Parameter(torch.from_numpy(param_values(case, i)).to(DEV, torch.bfloat16))
              for i in range(len(shapes))]
    opt = MSAM(params, base_optimizer=Lion, rho=rho, lr=g["lr"], betas=g["betas"], weight_decay=g["weight_decay"],
               momentum_dtype="int8")
    opt.inner.sr_seed = case["seed"]
    for step in range(1, case["steps"] + 1):
        for i, p in enumerate(params):
            p.grad = torch.from_numpy(grad_values(case, i, step)).to(DEV, torch.bfloat16)
        opt.step()
    opt.eval()
    evalp = [to_bits(p) for p in params]
    opt.train()
    torch.cuda.synchronize()
    assert opt._mnorm == oo.mnorm
    assert_same_as_oracle(case, oparams, params, opt, evalp=evalp, oeval=oeval, label="msam/lion")


def test_norm_is_bit_exact_on_sdxl_conv():
    """The norm over a large momentum set (the SDXL set's largest conv and a long
    1-D tensor): per-tensor sums of squares in the 64-lane order, then the fp32 fold."""
    from kaon_amd import MSAM

    print("[gpu] msam norm on a large conv", flush=True)
    shapes = [[1280, 1280, 3, 3], [1280], [640, 1280]]
    params = []
    for i, s in enumerate(shapes):
        gen = torch.Generator(device="cpu").manual_seed(100 + i)
        params.append(torch.nn.Parameter((torch.randn(*s, generator=gen) * 0.02).to(DEV, torch.bfloat16)))
    opt = MSAM(params, rho=0.3, lr=1e-3, momentum_dtype="int8")
    opt.inner.sr_seed = 1
    gen = torch.Generator(device="cpu").manual_seed(7)
    for p in params:
        p.grad = (torch.randn(*p.shape, generator=gen) * 1e-3).to(DEV, torch.bfloat16)
    opt.step()
    torch.cuda.synchronize()
    sq = np.float32(0.0)
    for i, p in enumerate(params):
        st = opt.inner.state[p]
        prm = O.make_param(tuple(p.shape), O.BF16, O.BF16, tensor_id=i,
                           p_values=np.zeros(p.shape, dtype=np.float32))
        prm.state["m"] = st["m"].cpu().numpy().reshape(-1).view(np.int8).reshape(st["m"].shape).copy()
        prm.state["m_scale"] = st["m_scale"].float().cpu().numpy().copy()
        t = O._tensor(prm, "int8")
        sq = np.float32(sq + np.float32(O.lib().ko_momentum_sumsq(ctypes.byref(t))))
    want = float(np.sqrt(sq, dtype=np.float32))
    assert opt._mnorm == want, (opt._mnorm, want)
    assert math.isfinite(want) and want > 0.0


def test_api_errors():
    from kaon_amd import MSAM

    p = torch.nn.Parameter(torch.zeros(8, 16, device=DEV, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        MSAM([p], norm="layer")
    with pytest.raises(ValueError):
        MSAM([p], eps=-1.0)
    opt = MSAM([p], rho=0.3)
    opt.eval()
    p.grad = torch.zeros_like(p)
    with pytest.raises(RuntimeError):
        opt.step()


def test_dtype_matrix_matches_oracle():
    """fp32 params with bf16 grads and the reverse."""
    for p, g in (("f32", "bf16"), ("bf16", "f32")):
        case = _case([[48, 40], [64]], dict(lr=1e-3, rho=0.3, momentum_dtype="int8"), p=p, g=g)
        print(f"[gpu] msam dtypes p={p} g={g}", flush=True)
        _check(case, f"p={p} g={g}")


@pytest.mark.parametrize("norm", ["global", "tensor", "none"])
@pytest.mark.parametrize("mom", ["bfloat16", "int8"])
def test_nan_momentum_follows_the_reference(norm, mom):
    """A NaN momentum coordinate (bf16) or row scale (int8) planted after two steps, then
    eval() / train().  norm="global" and "tensor" multiply the momentum by their scale with
    no sanitizing (msam.py:216-222): the global form carries the NaN coordinates into the
    weights, the tensor form makes its own norm NaN and so the whole tensor; norm="none"
    maps NaN to a zero climb (msam.py:223-230).  Weights must equal the oracle's bit for
    bit after each swap (a NaN bf16 weight is torch's 0x7FC0 on both sides)."""
    print(f"[gpu] msam NaN momentum norm={norm} mom={mom}", flush=True)
    case = _case([[24, 32], [40]], dict(lr=1e-3, rho=0.3, norm=norm, momentum_dtype=mom), steps=2, seed=11)
    case["eval_train"] = False
    oparams, oopt, _ = oracle_case_run(case)
    params, opt, _ = run_gpu(case)
    assert_same_as_oracle(case, oparams, params, opt, label=f"nan {norm} {mom} before")
    st = opt.inner.state[params[0]]
    if mom == "bfloat16":
        st["m"].view(torch.int16).view(-1)[5] = 0x7FC0
        oparams[0].state["m"].reshape(-1)[5] = 0x7FC0
    else:
        st["m_scale"].view(-1)[3] = float("nan")
        oparams[0].state["m_scale"].reshape(-1)[3] = np.float32("nan")
    for label, sign in (("eval", -1.0), ("train", +1.0)):
        if sign < 0:
            opt.eval()
        else:
            opt.train()
        oopt.msam_apply(sign)
        torch.cuda.synchronize()
        for i, (op, p) in enumerate(zip(oparams, params)):
            got, want = to_bits(p).reshape(-1), op.p.reshape(-1)
            assert np.array_equal(got, want), (norm, mom, label, i, int((got != want).sum()))
        w = O.bf16_to_f32(oparams[0].p.reshape(-1))
        nan_w = int(np.isnan(w).sum())
        if norm == "none":
            assert nan_w == 0
        elif norm == "tensor":
            assert nan_w == w.size
        else:
            assert nan_w == (1 if mom == "bfloat16" else 32)
