"""AdaPNM on the GPU against the oracle, bit for bit.

The oracle's AdaPNM (oracle/kaon_oracle.c ko_adapnm_tensor) matches the
reference's own output on the golden cases (tests/test_oracle_golden.py).
Here the HIP step (kaon_adapnm_step through kaon_amd.AdaPNM) must reproduce the
oracle exactly: weights, both momentum buffers (codes and scales), the
factored / 1-D second moment, max_v and the kahan shift, over several steps
so that each buffer is the positive one more than once.  Extra cases cover
what the golden ones do not: rows long enough for several runs, ragged rows
(C % 8 != 0, the scalar path), 4-bit blocks spanning rows, fp32 params with
bf16 grads and the reverse, AMSBound, clip 0, no cautious / no GC, rows the
specialized keep-count / apply kernel takes (every codec, with and without
weight decay), and the SDXL set's largest conv.
"""
import io

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

import oracle as O  # noqa: E402
from cases import grad_values  # noqa: E402
from golden_compare import CASES, group_for, load_golden  # noqa: E402
from gpu_cases import DEV, assert_same_as_oracle, make_opt, oracle_case_run, run_gpu, tdtype  # noqa: E402

GOLDEN = [k for k, c in CASES.items() if c["opt"] == "adapnm"]


@pytest.fixture(autouse=True, scope="module")
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")


@pytest.mark.parametrize("name", GOLDEN)
def test_golden_case_bit_exact(name):
    case = CASES[name]
    print(f"[gpu] adapnm golden {name}", flush=True)
    oparams, _oopt, _ = oracle_case_run(case)
    params, opt, _ = run_gpu(case)
    assert_same_as_oracle(case, oparams, params, opt, label=name)


def _case(shapes, kwargs, steps=4, p="bf16", g="bf16", seed=11):
    return dict(steps=steps, seed=seed, p_dtype=p, g_dtype=g, opt="adapnm", shapes=shapes, kwargs=kwargs)


EXTRA = {
    # several runs per tensor (R > 16 * rows per wave), int8 and 4-bit, SR
    "runs_int8": _case([[640, 64], [300, 72], [5120]], dict(lr=1e-3, momentum_dtype="int8", weight_decay=0.05)),
    "runs_4bit_b64": _case([[160, 40], [96, 24, 3, 3], [1000]], dict(lr=1e-3, momentum_dtype="4bit",
                                                                      momentum_4bit_block=64, beta0=1.0)),
    # ragged rows: C % 8 != 0, odd 1-D length, 4-bit blocks straddling rows
    "ragged_4bit": _case([[37, 45], [13, 7, 3], [101], [5, 3]], dict(lr=1e-3, momentum_dtype="4bit",
                                                                      momentum_4bit_block=16)),
    "ragged_bf16_rn": _case([[37, 45], [101], [9, 11]], dict(lr=2e-3, momentum_dtype="bfloat16",
                                                             bf16_method="none", weight_decay=0.1)),
    # mixed dtypes
    "f32p_bf16g": _case([[48, 40], [64]], dict(lr=1e-3, momentum_dtype="int8"), p="f32", g="bf16"),
    "bf16p_f32g": _case([[48, 40], [64]], dict(lr=1e-3, momentum_dtype="float32"), p="bf16", g="f32"),
    # AMSBound on 1-D, clip 0 (no clip), cautious and GC off, kahan
    "ams_noclip": _case([[24, 32], [80], [33]], dict(lr=1e-3, momentum_dtype="bfloat16", ams_bound=True,
                                                     clip_threshold=0.0, cautious=False,
                                                     gradient_centralization=False)),
    "kahan_int8": _case([[40, 24], [56]], dict(lr=1e-3, momentum_dtype="int8", bf16_method="kahan")),
    "beta1_zero": _case([[32, 16], [20]], dict(lr=1e-3, betas=(0.0, 0.99), momentum_dtype="bfloat16")),
    # rows the specialized keep-count / apply kernel takes (bf16 p and g, SR, C % 8 == 0,
    # 4-bit blocks tiling the rows), each buffer positive twice
    "fast_4bit_b128": _case([[256, 2048], [128, 128, 3, 3], [96]], dict(lr=1e-3, momentum_dtype="4bit",
                                                                        momentum_4bit_block=128)),
    "fast_bf16_wd": _case([[320, 1280], [64, 640]], dict(lr=1e-3, momentum_dtype="bfloat16", weight_decay=0.1)),
    "fast_int8_noclip": _case([[200, 512], [48, 32, 3, 3]], dict(lr=2e-3, momentum_dtype="int8", clip_threshold=0.0,
                                                                 beta0=1.0)),
    # rows of 5 to 10 chunks per lane (the prefetching clip-sum kernel's second row class)
    "class1_int8": _case([[96, 5120], [64, 320, 3, 3], [40, 2056]], dict(lr=1e-3, momentum_dtype="int8")),
    "class1_bf16": _case([[48, 4096], [32, 2880]], dict(lr=1e-3, momentum_dtype="bfloat16", weight_decay=0.01)),
    # fp16 params and grads (the reference's native path: p.mul_(1 - lr*wd) and subtract_one_ in
    # fp16, RN under "stochastic_rounding", src/kaon/adapnm.py:1222-1258, src/kaon/_backend.py:82-98)
    "f16_int8_sr": _case([[40, 24], [16, 8, 3, 3], [56]], dict(lr=1e-3, momentum_dtype="int8", weight_decay=0.05),
                         p="f16", g="f16"),
    "f16_4bit_kahan": _case([[37, 45], [101]], dict(lr=1e-3, momentum_dtype="4bit", momentum_4bit_block=16,
                                                    bf16_method="kahan", weight_decay=0.1), p="f16", g="f16"),
    "f16_bf16_rn_ams": _case([[48, 40], [80]], dict(lr=2e-3, momentum_dtype="bfloat16", bf16_method="none",
                                                    ams_bound=True), p="f16", g="f16"),
}


@pytest.mark.parametrize("name", sorted(EXTRA))
def test_extra_case_bit_exact(name):
    case = EXTRA[name]
    print(f"[gpu] adapnm extra {name}", flush=True)
    oparams, _oopt, _ = oracle_case_run(case)
    params, opt, _ = run_gpu(case)
    assert_same_as_oracle(case, oparams, params, opt, label=name)


def test_sdxl_largest_conv_two_steps():
    """[1280, 1280, 3, 3] (C = 11520, 14.7M elements), int8 momenta: the SDXL set's
    largest tensor, through the streamed row class."""
    case = _case([[1280, 1280, 3, 3]], dict(lr=1e-4, momentum_dtype="int8"), steps=2, seed=3)
    print("[gpu] adapnm conv1280 x2", flush=True)
    oparams, _oopt, _ = oracle_case_run(case)
    params, opt, _ = run_gpu(case)
    assert_same_as_oracle(case, oparams, params, opt, label="conv1280")


def test_save_load_resume_matches_uninterrupted():
    """3 steps, torch.save / torch.load (weights_only) into a fresh optimizer, 2
    more: identical to 5 uninterrupted steps (the group step, and with it the
    buffer alternation and the bias corrections, round-trips)."""
    case = dict(CASES["pnm_int8_sr"])
    print("[gpu] adapnm save/load resume", flush=True)
    ref_params, ref_opt, _ = run_gpu(dict(case, steps=5))
    params, opt, _ = run_gpu(dict(case, steps=3))
    buf = io.BytesIO()
    torch.save(opt.state_dict(), buf)
    buf.seek(0)
    sd = torch.load(buf, weights_only=True)
    assert sd["param_groups"][0]["step"] == 3
    params2 = [torch.nn.Parameter(p.detach().clone()) for p in params]
    opt2 = make_opt(case, params2)
    opt2.load_state_dict(sd)
    gdt = tdtype(case["g_dtype"])
    for step in (4, 5):
        for i, p in enumerate(params2):
            p.grad = torch.from_numpy(grad_values(case, i, step)).to(DEV, gdt)
        opt2.step()
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(ref_params, params2)):
        assert torch.equal(a.detach().view(torch.int16), b.detach().view(torch.int16)), (i, "weights")
        sa, sb = ref_opt.state[a], opt2.state[b]
        for k in sa:
            if torch.is_tensor(sa[k]):
                assert torch.equal(sa[k].reshape(-1).view(torch.uint8), sb[k].reshape(-1).view(torch.uint8)), (i, k)
            else:
                assert sa[k] == sb[k], (i, k)


def _golden_state(gold, i):
    pre = f"s{i}_"
    return {k[len(pre):]: a for k, a in gold.items() if k.startswith(pre)}


@pytest.mark.parametrize("name", GOLDEN)
def test_resume_from_reference_checkpoint(name):
    """The reference's own state after its steps (the golden fixture), loaded in
    the reference's layout with the group's step count, then one more step on
    the GPU and in the oracle from the same params and state: identical.  The
    step count decides which buffer is positive and the bias corrections."""
    case = CASES[name]
    print(f"[gpu] adapnm resume from reference checkpoint {name}", flush=True)
    gold = load_golden(name)
    pdt, gdt = tdtype(case["p_dtype"]), tdtype(case["g_dtype"])
    steps, nxt = case["steps"], case["steps"] + 1

    def tensor_of(a, dt):
        if dt == torch.bfloat16:
            return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
        return torch.from_numpy(a.astype(np.float32) if a.dtype == np.float32 else a.copy())

    params = [torch.nn.Parameter(tensor_of(gold[f"p{i}"], pdt).to(DEV)) for i in range(len(case["shapes"]))]
    opt = make_opt(case, params)
    sd = opt.state_dict()
    sd.pop("kaon_amd", None)
    sd["param_groups"][0]["step"] = steps
    st = {}
    for i in range(len(params)):
        st[i] = {}
        for k, a in _golden_state(gold, i).items():
            if k.endswith("_numel") or k.endswith("_block"):
                st[i][k] = int(a)
            else:
                st[i][k] = tensor_of(a, torch.bfloat16 if a.dtype == np.uint16 else None)
    sd["state"] = st
    opt.load_state_dict(sd)
    for i, p in enumerate(params):
        p.grad = torch.from_numpy(grad_values(case, i, nxt)).to(DEV, gdt)
    opt.step()
    torch.cuda.synchronize()
    dt = O.BF16 if case["p_dtype"] == "bf16" else O.F32
    gt = O.BF16 if case["g_dtype"] == "bf16" else O.F32
    oparams = [O.make_param(shape, dt, gt, tensor_id=i, p_values=O.values(gold[f"p{i}"], dt))
               for i, shape in enumerate(case["shapes"])]
    oopt = O.OracleOptimizer(oparams, "adapnm", group_for(case), seed=case["seed"])
    oopt.t = steps
    for i, prm in enumerate(oparams):
        for k, a in _golden_state(gold, i).items():
            if k.endswith("_numel") or k.endswith("_block"):
                prm.state[k] = int(a)
            else:
                prm.state[k] = np.ascontiguousarray(a).reshape(np.shape(prm.state[k])).copy()
        g = grad_values(case, i, nxt)
        prm.g = O.f32_to_bf16(g).reshape(prm.shape) if gt == O.BF16 else g.copy()
    oopt.step()
    assert opt.param_groups[0]["step"] == nxt
    assert_same_as_oracle(case, oparams, params, opt, label=f"resume {name}")
