"""KProdigy on the GPU against the oracle, bit for bit.

The oracle's KProdigy (oracle/kaon_oracle.c ko_kprodigy_pass1_tensor /
ko_kprodigy_pass2_tensor, the D update in oracle/oracle.py) matches the
reference's own output on the golden cases (tests/test_oracle_golden.py).  Here
the HIP passes with the host-side D update (kaon_amd.KProdigy) must reproduce
the oracle exactly: the D estimate after every step (the per-tensor statistics
are FSUMs computed in the same order on both sides and folded identically),
weights, momentum codes and scales, v / row / col, s, p0 and the per-param
step.  Extra cases: tensors with more than one statistics block (the flat sum
across blocks), slice_p > 1 over ragged lengths, 1-D params, fp32/bf16 mixes,
two param groups with independent and with shared D, a frozen (lr 0) group in
a shared scope, and the SDXL set's largest conv.
"""
import io

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

import oracle as O  # noqa: E402
from cases import grad_values, param_values  # noqa: E402
from golden_compare import CASES, dt, group_for  # noqa: E402
from gpu_cases import DEV, assert_same_as_oracle, make_opt, oracle_case_run, run_gpu, tdtype  # noqa: E402

GOLDEN = [k for k, c in CASES.items() if c["opt"] == "kprodigy"]


@pytest.fixture(autouse=True, scope="module")
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")


def _run_both(case):
    """Step the GPU and the oracle side by side; D must agree after every step."""
    gparams, gopt, _ = run_gpu(dict(case, steps=0))
    oparams, oopt, _ = oracle_case_run(dict(case, steps=0))
    gdt = tdtype(case["g_dtype"])
    for step in range(1, case["steps"] + 1):
        for i, (p, op) in enumerate(zip(gparams, oparams)):
            g = grad_values(case, i, step)
            p.grad = torch.from_numpy(g).to(DEV, gdt)
            if op.g_dtype == O.BF16:
                op.g = O.f32_to_bf16(g).reshape(op.shape)
            elif op.g_dtype == O.F16:
                op.g = O.f32_to_f16(g).reshape(op.shape)
            else:
                op.g = g.copy()
        gopt.step()
        oopt.step()
        assert gopt.param_groups[0]["d"] == oopt.group["d"], (step, gopt.param_groups[0]["d"], oopt.group["d"])
        assert gopt.param_groups[0]["d_max"] == oopt.group["d_max"]
        assert gopt.param_groups[0]["k"] == oopt.group["k"]
    torch.cuda.synchronize()
    return gparams, gopt, oparams, oopt


@pytest.mark.parametrize("name", GOLDEN)
def test_golden_case_bit_exact(name):
    case = CASES[name]
    print(f"[gpu] kprodigy golden {name}", flush=True)
    gparams, gopt, oparams, _ = _run_both(case)
    assert_same_as_oracle(case, oparams, gparams, gopt, label=name)


def _case(shapes, kwargs, steps=4, p="bf16", g="bf16", seed=21):
    return dict(steps=steps, seed=seed, p_dtype=p, g_dtype=g, opt="kprodigy", shapes=shapes, kwargs=kwargs)


EXTRA = {
    # 40000 and 50000 sliced elements: three and four statistics blocks of 16384
    "blocks_full": _case([[200, 200], [50000], [37, 45]], dict(lr=1.0, momentum_dtype="int8", cautious=True)),
    "blocks_slice7": _case([[640, 300], [13, 7, 3]], dict(lr=1.0, momentum_dtype="4bit", momentum_4bit_block=64,
                                                          slice_p=7, weight_decay=0.01)),
    "factored_slice3": _case([[96, 48], [32, 16, 3, 3], [77]], dict(lr=1.0, second_moment="factored",
                                                                    momentum_dtype="bfloat16", slice_p=3,
                                                                    weight_decay=0.05, cautious=True)),
    "f32p_bf16g": _case([[48, 40], [64]], dict(lr=1.0, momentum_dtype="float32", decouple=False,
                                               weight_decay=0.1), p="f32", g="bf16"),
    "bf16p_f32g_rn": _case([[48, 40], [64]], dict(lr=1.0, momentum_dtype="int8", bf16_method="none",
                                                  use_bias_correction=True), p="bf16", g="f32"),
    "nomom_growth": _case([[64, 32], [33]], dict(lr=1.0, betas=(0.0, 0.99), growth_rate=1.02, d_coef=2.0,
                                                 safeguard_warmup=True), steps=6),
    # the factored second moment of the decayed gradient fma(wd, p, GC(g)) (_collect_grad,
    # kprodigy.py:406-414): every row class (prefetching-class rows on the register kernel,
    # ragged rows, a row of the widest class, a streamed row of 2500 chunks), int8 momentum
    "factored_coupled": _case([[96, 48], [32, 16, 3, 3], [33, 45], [40, 1280], [6, 11520], [4, 20000], [77]],
                              dict(lr=1.0, second_moment="factored", momentum_dtype="int8", decouple=False,
                                   weight_decay=0.1, cautious=True), steps=3),
    # fp16 params and grads (RN under "stochastic_rounding", kahan in fp16): full and factored v
    "f16_full_sr": _case([[48, 40], [16, 8, 3, 3], [70]], dict(lr=1.0, momentum_dtype="int8", weight_decay=0.01,
                                                              cautious=True), p="f16", g="f16"),
    "f16_factored_kahan": _case([[64, 48], [33, 45], [20]], dict(lr=1.0, second_moment="factored",
                                                                 momentum_dtype="bfloat16", bf16_method="kahan",
                                                                 decouple=False, weight_decay=0.05),
                                p="f16", g="f16"),
    # factor_conv_as_matrix=False: the second moment of the 3-D / 4-D weights factored over
    # their last two dims, each [kh, kw] block on its own (k_pd_bfac)
    "blockfac_int8": _case([[16, 8, 3, 3], [6, 5, 4], [32, 24], [20]],
                           dict(lr=1.0, second_moment="factored", factor_conv_as_matrix=False,
                                momentum_dtype="int8", cautious=True, weight_decay=0.01), steps=3),
    "blockfac_coupled_f32p": _case([[8, 4, 5, 3], [12, 10]],
                                   dict(lr=1.0, second_moment="factored", factor_conv_as_matrix=False,
                                        momentum_dtype="4bit", momentum_4bit_block=16, decouple=False,
                                        weight_decay=0.05), p="f32", g="bf16", steps=3),
    "blockfac_sdxl_conv": _case([[320, 320, 3, 3]], dict(lr=1.0, second_moment="factored",
                                                         factor_conv_as_matrix=False, momentum_dtype="bfloat16"),
                                steps=2),
    # fp32 params under the coupled decay, bf16 grads, 4-bit momentum, no GC
    "factored_coupled_f32p": _case([[64, 40], [16, 8, 3, 3], [50]],
                                   dict(lr=1.0, second_moment="factored", momentum_dtype="4bit",
                                        momentum_4bit_block=32, decouple=False, weight_decay=0.05,
                                        gradient_centralization=False), p="f32", g="bf16", steps=3),
}


@pytest.mark.parametrize("name", sorted(EXTRA))
def test_extra_case_bit_exact(name):
    case = EXTRA[name]
    print(f"[gpu] kprodigy extra {name}", flush=True)
    gparams, gopt, oparams, _ = _run_both(case)
    assert_same_as_oracle(case, oparams, gparams, gopt, label=name)


def test_sdxl_largest_conv_three_steps():
    case = _case([[1280, 1280, 3, 3]], dict(lr=1.0, momentum_dtype="int8"), steps=3, seed=5)
    print("[gpu] kprodigy conv1280 x3", flush=True)
    gparams, gopt, oparams, _ = _run_both(case)
    assert_same_as_oracle(case, oparams, gparams, gopt, label="conv1280")


def _two_group_run(independent, lrs, steps=4):
    """Two param groups stepped on the GPU and, group by group with the scope's
    shared D, in the oracle; returns (gpu groups, oracle D per group)."""
    case = _case([[40, 24], [56], [24, 20]], dict(lr=1.0, momentum_dtype="bfloat16"), steps=steps, seed=31)
    from kaon_amd import KProdigy

    pdt = tdtype(case["p_dtype"])
    params = [torch.nn.Parameter(torch.from_numpy(param_values(case, i)).to(DEV, pdt)) for i in range(3)]
    opt = KProdigy([{"params": params[:2], "lr": lrs[0]}, {"params": params[2:], "lr": lrs[1]}],
                   independent_d=independent)
    opt.sr_seed = case["seed"]
    for step in range(1, steps + 1):
        for i, p in enumerate(params):
            p.grad = torch.from_numpy(grad_values(case, i, step)).to(DEV, pdt)
        opt.step()
    torch.cuda.synchronize()
    return opt, params, case


def test_two_groups_independent_d_match_single_group_runs():
    """independent_d: each group is its own D scope, so each matches a
    one-group run over its own params (same tensor ids, same SR key)."""
    opt, params, case = _two_group_run(True, (1.0, 0.5))
    print("[gpu] kprodigy two groups independent", flush=True)
    for gi, (idx, lr) in enumerate((([0, 1], 1.0), ([2], 0.5))):
        oparams = [O.make_param(case["shapes"][i], O.BF16, O.BF16, tensor_id=i, p_values=param_values(case, i))
                   for i in idx]
        oopt = O.OracleOptimizer(oparams, "kprodigy", dict(group_for(case), lr=lr), seed=case["seed"])
        for step in range(1, case["steps"] + 1):
            for prm, i in zip(oparams, idx):
                prm.g = O.f32_to_bf16(grad_values(case, i, step)).reshape(prm.shape)
            oopt.step()
        assert opt.param_groups[gi]["d"] == oopt.group["d"], gi
        for prm, i in zip(oparams, idx):
            got = params[i].detach().view(torch.int16).cpu().numpy().view(np.uint16)
            assert np.array_equal(got, prm.p), (gi, i)


def test_shared_d_with_a_frozen_group():
    """A shared scope whose second group has lr 0 (kprodigy.py:330-334): its
    params skip the D statistics, D comes from the first group alone and both
    groups carry the same D."""
    opt, params, case = _two_group_run(False, (1.0, 0.0))
    print("[gpu] kprodigy shared d, frozen group", flush=True)
    assert opt.param_groups[0]["d"] == opt.param_groups[1]["d"]
    with pytest.raises(RuntimeError, match="same lr"):
        _two_group_run(False, (1.0, 0.5), steps=1)


def test_save_load_resume_matches_uninterrupted():
    case = dict(CASES["pd_int8_factored"])
    print("[gpu] kprodigy save/load resume", flush=True)
    ref_params, ref_opt, _ = run_gpu(dict(case, steps=5))
    params, opt, _ = run_gpu(dict(case, steps=3))
    buf = io.BytesIO()
    torch.save(opt.state_dict(), buf)
    buf.seek(0)
    sd = torch.load(buf, weights_only=True)
    params2 = [torch.nn.Parameter(p.detach().clone()) for p in params]
    opt2 = make_opt(case, params2)
    opt2.load_state_dict(sd)
    assert opt2.param_groups[0]["d"] == opt.param_groups[0]["d"]
    gdt = tdtype(case["g_dtype"])
    for step in (4, 5):
        for i, p in enumerate(params2):
            p.grad = torch.from_numpy(grad_values(case, i, step)).to(DEV, gdt)
        opt2.step()
    torch.cuda.synchronize()
    assert opt2.param_groups[0]["d"] == ref_opt.param_groups[0]["d"]
    for i, (a, b) in enumerate(zip(ref_params, params2)):
        assert torch.equal(a.detach().view(torch.int16), b.detach().view(torch.int16)), (i, "weights")
        sa, sb = ref_opt.state[a], opt2.state[b]
        for k in sa:
            if torch.is_tensor(sa[k]):
                assert torch.equal(sa[k].reshape(-1).view(torch.uint8), sb[k].reshape(-1).view(torch.uint8)), (i, k)
            else:
                assert sa[k] == sb[k], (i, k)
