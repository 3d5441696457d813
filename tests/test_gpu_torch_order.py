"""The HIP step with reduction_order="torch" against the reference's own output.

In this mode the step's fp32 sums -- the GC row means, the factored row and
column means, the row factors' mean, the RMS clip's norm (eight sequential fma
chains) and MSAM norm="tensor"'s per-tensor momentum norm -- run in torch CPU's
order (kaon_torch.hip).  The fixtures under tests/golden/ hold the reference's
weights and state, written by kaon 0.7.4 on torch CPU with the library's Philox
noise injected into its stochastic rounding (tests/golden/make_golden.py), so
the GPU is compared with them directly:

* configs[0] (Adakaon, conv [320,320,3,3] + linear [1280,1280], SR, 10 steps):
  the SHA-256 of both params' bf16 bits equals the reference's after every step,
  and the factored state equals the reference's bit for bit;
* every bf16 / fp16 golden case of Adakaon, Lion, Nekaon and MSAM norm="none" /
  "tensor": no weight differs (eval-mode weights included), momentum codes are
  equal, scales within 1 fp32 ulp, fp32 state within 1e-6 relative (north
  star's bars); in fact the state is checked equal to the bit;
* the fp32-grad cases: weights, momentum and state equal to the reference's;
* every case and a set of larger and ragged shapes also bit for bit against the
  oracle run in torch order (oracle.torch_order()).
"""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

import oracle as O  # noqa: E402
from cases import grad_values, param_values  # noqa: E402
from golden_compare import CASES, CFG0, bf16_mismatch, load_golden, rel_err  # noqa: E402
from gpu_cases import DEV, assert_same_as_oracle, oracle_case_run, run_gpu, state_of, to_bits  # noqa: E402
from measure_budgets import f32_ulps  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
TORCH = {"reduction_order": "torch"}
_MOM = ("m",)


def _torch_case(c):
    if c["opt"] in ("adakaon", "lion", "nekaon"):
        return True
    return c["opt"] == "msam" and c["kwargs"].get("norm", "global") in ("none", "tensor")


BIT = sorted(k for k, c in CASES.items() if _torch_case(c) and c["g_dtype"] in ("bf16", "f16"))
F32 = sorted(k for k, c in CASES.items() if _torch_case(c) and c["g_dtype"] == "f32")


@pytest.fixture(autouse=True, scope="module")
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")


def test_cfg0_per_step_hashes_equal_the_reference():
    """after each of the 10 steps the SHA-256 of both params' bf16 bits is
    the reference's (tests/golden/golden_meta.json); the final row / col are its bits."""
    print("[gpu] torch order: configs[0], 10 steps", flush=True)
    from kaon_amd import Adakaon

    want = json.load(open(os.path.join(HERE, "golden", "golden_meta.json")))["cases"]["cfg0"]["hashes"]
    gold = load_golden("cfg0")
    params = [torch.nn.Parameter(torch.from_numpy(param_values(CFG0, i)).to(DEV, torch.bfloat16))
              for i in range(len(CFG0["shapes"]))]
    opt = Adakaon(params, lr=1e-4, betas=(0.0, 0.999), bf16_method="stochastic_rounding", reduction_order="torch")
    opt.sr_seed = CFG0["seed"]
    for step in range(1, CFG0["steps"] + 1):
        for i, p in enumerate(params):
            p.grad = torch.from_numpy(grad_values(CFG0, i, step)).to(DEV, torch.bfloat16)
        opt.step()
        got = hashlib.sha256(b"".join(np.ascontiguousarray(to_bits(p)).tobytes() for p in params)).hexdigest()
        assert got == want[step - 1], f"step {step}: weights differ from the reference's"
    for i, p in enumerate(params):
        for k in ("row", "col"):
            a = opt.state[p][k].cpu().numpy().view(np.uint32)
            b = gold[f"s{i}_{k}"].reshape(-1).view(np.uint32)
            assert np.array_equal(a, b), (i, k, int((a != b).sum()))


def _gold_compare_bits(name, params, opt, evalp):
    gold = load_golden(name)
    for i, p in enumerate(params):
        nm, mu = bf16_mismatch(to_bits(p), gold[f"p{i}"])  # 16-bit patterns (bf16 or fp16)
        assert nm == 0, f"{name} param {i}: {nm} weights differ from the reference's (max {mu} ulp)"
        if evalp is not None:
            e = evalp[i].reshape(-1)
            nm = int((e != gold[f"p{i}_eval"].reshape(-1)).sum())
            assert nm == 0, f"{name} param {i}: {nm} eval-mode weights differ"
        st = state_of(opt, p)
        for k in ("row", "col", "v"):
            if f"s{i}_{k}" in gold:
                a = st[k].cpu().numpy().reshape(-1)
                b = gold[f"s{i}_{k}"].reshape(-1)
                assert rel_err(a, b) <= 1e-6, (name, i, k)
                assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (name, i, k)
        for k in _MOM:
            if k not in st:
                continue
            a, b = to_bits(st[k]).reshape(-1), gold[f"s{i}_{k}"].reshape(-1)
            if a.dtype != b.dtype and a.itemsize == b.itemsize:
                a = a.view(b.dtype)
            assert np.array_equal(a, b), f"{name} param {i}: {int((a != b).sum())} momentum codes differ"
            if f"{k}_scale" in st:
                ulps = f32_ulps(st[f"{k}_scale"].cpu().numpy(), gold[f"s{i}_{k}_scale"])
                assert ulps <= 1, (name, i, ulps)


@pytest.mark.parametrize("name", BIT)
def test_low_precision_case_equals_the_reference(name):
    print(f"[gpu] torch order: golden {name}", flush=True)
    case = CASES[name]
    params, opt, evalp = run_gpu(case, extra=TORCH)
    _gold_compare_bits(name, params, opt, evalp)
    with O.torch_order():
        oparams, _oopt, oeval = oracle_case_run(case)
    assert_same_as_oracle(case, oparams, params, opt, evalp=evalp, oeval=oeval, label=name)


@pytest.mark.parametrize("name", F32)
def test_fp32_grad_case_equals_the_reference(name):
    print(f"[gpu] torch order: golden {name}", flush=True)
    case = CASES[name]
    gold = load_golden(name)
    params, opt, evalp = run_gpu(case, extra=TORCH)
    for i, p in enumerate(params):
        a = p.detach().cpu().numpy().reshape(-1)
        assert np.array_equal(a.view(np.uint32), gold[f"p{i}"].reshape(-1).view(np.uint32)), (name, i)
        if evalp is not None:
            assert np.array_equal(evalp[i].reshape(-1).view(np.uint32),
                                  gold[f"p{i}_eval"].reshape(-1).view(np.uint32)), (name, i, "eval")
        st = state_of(opt, p)
        for k in ("row", "col", "v", "m"):
            if f"s{i}_{k}" not in gold or k not in st:
                continue
            a, b = to_bits(st[k]).reshape(-1), gold[f"s{i}_{k}"].reshape(-1)
            if a.dtype != b.dtype and a.itemsize == b.itemsize:
                a = a.view(b.dtype)
            assert np.array_equal(a, b), (name, i, k, int((a != b).sum()))
    with O.torch_order():
        oparams, _oopt, oeval = oracle_case_run(case)
    assert_same_as_oracle(case, oparams, params, opt, evalp=evalp, oeval=oeval, label=name)


def _case(opt, shapes, kwargs, steps=2, p="bf16", g="bf16", seed=21, **kw):
    c = dict(steps=steps, seed=seed, p_dtype=p, g_dtype=g, opt=opt, shapes=shapes, kwargs=kwargs)
    c.update(kw)
    return c


EXTRA = {
    # the set's largest conv and linear shapes (rows of 11520 and 1280 elements, 5120 rows)
    "sdxl_conv_int8": _case("adakaon", [[1280, 1280, 3, 3], [1280]],
                            dict(lr=1e-4, betas=(0.9, 0.999), momentum_dtype="int8"), steps=1),
    "sdxl_linear_4bit": _case("adakaon", [[5120, 1280], [640, 2048], [5120]],
                              dict(lr=1e-4, betas=(0.9, 0.999), momentum_dtype="4bit", weight_decay=0.1)),
    # column sums in every torch form: 32-column blocks plus an 8-block and single
    # columns (C = 45, 77), C < 8 (4-blocks and singles), rows shorter than 8, row
    # counts that are not multiples of 4 or 16; ragged chunks in the clip
    "ragged_bf16": _case("adakaon", [[37, 45], [19, 77], [40, 5], [9, 3], [13, 7, 3], [101], [5]],
                         dict(lr=2e-3, betas=(0.9, 0.999), momentum_dtype="bfloat16"), steps=3),
    "ragged_rn_nogc": _case("adakaon", [[300, 72], [33, 250], [1000]],
                            dict(lr=1e-3, betas=(0.8, 0.99), momentum_dtype="int8", bf16_method="none",
                                 gradient_centralization=False, cautious=False), steps=3),
    # many rows (the cascade's second level) and long 1-D tensors (rows of > 2^16 terms)
    # column sums at four columns per lane (1536 < R <= 3072), 2048 rows with int8
    # codes and 1600 rows of 96 columns
    "mid_rows_bf16": _case("adakaon", [[2048, 640], [1600, 96], [640]],
                           dict(lr=1e-4, betas=(0.9, 0.999), momentum_dtype="int8", weight_decay=0.01)),
    "tall_f32": _case("adakaon", [[4100, 40], [70000]],
                      dict(lr=1e-3, betas=(0.9, 0.999), momentum_dtype="float32", weight_decay=0.01),
                      p="f32", g="f32"),
    "lion_ragged": _case("lion", [[77, 33], [640, 45], [129]],
                         dict(lr=2e-4, betas=(0.95, 0.98), momentum_dtype="int8"), steps=3),
    "nekaon_sdxl": _case("nekaon", [[640, 640, 3, 3], [1280, 5120]],
                         dict(lr=1e-4, k=1.5, betas=(0.2, 0.999), momentum_dtype="4bit",
                              momentum_4bit_block=64), steps=2, eval_train=True, outlier_frac=0.01),
    "f16_sr": _case("adakaon", [[96, 200], [48, 16, 3, 3], [300]],
                    dict(lr=1e-3, betas=(0.9, 0.999), momentum_dtype="int8"), p="f16", g="f16"),
    "msam_tensor_bf16": _case("msam", [[320, 1280], [77, 33], [640]],
                              dict(lr=1e-3, rho=0.3, norm="tensor", momentum_dtype="bfloat16"), steps=2,
                              eval_train=True),
}


@pytest.mark.parametrize("name", sorted(EXTRA))
def test_extra_case_bit_exact_against_oracle_in_torch_order(name):
    print(f"[gpu] torch order: extra {name}", flush=True)
    case = EXTRA[name]
    params, opt, evalp = run_gpu(case, extra=TORCH)
    with O.torch_order():
        oparams, _oopt, oeval = oracle_case_run(case)
    assert_same_as_oracle(case, oparams, params, opt, evalp=evalp, oeval=oeval, label=name)


def test_long_chain_split_matches_one_stream(monkeypatch):
    """The torch-order step with the long tensors' clip chains on the side stream
    (KaonLaunch.n_long > 0) against the same steps with every kernel on the launch
    stream (n_long forced to 0): equal weights, codes, scales and state, bit for bit.
    Two long convs (14.7 M and 7.4 M elements: both at least half the largest), short
    matrices and 1-D vectors, so the split covers specialized and generic items
    on both sides; Nekaon adds the removal and the climb."""
    print("[gpu] torch order: long-chain split against one stream", flush=True)
    from kaon_amd import _engine as E

    shapes = [[1280, 1280, 3, 3], [640, 1280, 3, 3], [1280, 1280], [320, 2880], [5120], [1000]]
    for name, kw in (("adakaon", dict(lr=1e-4, betas=(0.9, 0.999), momentum_dtype="int8")),
                     ("nekaon", dict(lr=1e-4, k=1.5, betas=(0.2, 0.999), momentum_dtype="4bit",
                                     momentum_4bit_block=64))):
        case = _case(name, shapes, kw, steps=2, seed=31)
        split_params, split_opt, _ = run_gpu(case, extra=TORCH)
        inner = getattr(split_opt, "inner", split_opt)
        plans = [pl for _key, (_ptrs, pl) in inner._plans.items()]
        assert plans and max(pl.launch.n_long for pl in plans) == 2, [pl.launch.n_long for pl in plans]

        class OneStreamPlan(E.Plan):
            def __init__(self, *a, **k):
                super().__init__(*a, **k)
                self.launch.n_long = 0

        monkeypatch.setattr(E, "Plan", OneStreamPlan)
        one_params, one_opt, _ = run_gpu(case, extra=TORCH)
        monkeypatch.undo()
        for i, (a, b) in enumerate(zip(split_params, one_params)):
            assert np.array_equal(to_bits(a), to_bits(b)), (name, i)
            sa, sb = state_of(split_opt, a), state_of(one_opt, b)
            for k in sa:
                if torch.is_tensor(sa[k]):
                    assert np.array_equal(to_bits(sa[k]), to_bits(sb[k])), (name, i, k)
