"""p.grad after a step with gradient centralization.

The reference's native paths (Adakaon / AdaPNM with fused=False, and Lion,
AdaMuon, KProdigy, which have no fused path) centralize p.grad in place
before stepping (centralize_grads_, src/kaon/_backend.py:147-177), so a
caller reading p.grad after step() sees g - mean over the fan-in, in the
grad dtype, for params of 2 dims or more.  The fused Adakaon / AdaPNM kernels
centralize in-kernel and leave p.grad as it was (src/kaon/adakaon.py:387-409);
the fused Adakaon still sends some params to its native path (fp16, convs with
quantized momentum, beta1 = 0, bf16 without SR, one-block 4-bit matrices of odd
width: _fused_partition, adakaon.py:437-468), whose p.grad it centralizes.
The Adakaon / Lion apply (Nekaon's and MSAM's removal / climb applies
included) and KProdigy's pass 2 store the centralized gradient as they read it
(KAON_F_GC_WRITE); AdaPNM and AdaMuon write it back after the step with
kaon_gc_writeback.  Checked against the oracle's bf16 GC, after the last of
the case's steps (Nekaon and MSAM: the second, whose apply carries the removal).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

import oracle as O  # noqa: E402
from cases import grad_values, param_values  # noqa: E402
from gpu_cases import DEV, make_opt, to_bits  # noqa: E402

SHAPES = [[24, 40], [16, 8, 3, 3], [33], [7, 9]]


@pytest.fixture(autouse=True, scope="module")
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")


def _case(opt, steps=1, **kw):
    return dict(steps=steps, seed=5, p_dtype="bf16", g_dtype="bf16", opt=opt, shapes=SHAPES, kwargs=kw)


ALL = True
FUSED = {"fused": True}
# case, the indices of SHAPES whose p.grad is left centralized (ALL: every param of
# 2 dims or more), constructor extras
CASES = {
    "adakaon_native": (_case("adakaon", lr=1e-3, momentum_dtype="int8"), ALL, None),
    # fused, int8: the conv goes native (quantized conv momentum), the matrices one-block
    "adakaon_fused": (_case("adakaon", lr=1e-3, momentum_dtype="int8"), {1}, FUSED),
    # fused, bf16 momentum: every matrix and the conv run one-block
    "adakaon_fused_bf16": (_case("adakaon", lr=1e-3, momentum_dtype="bfloat16"), set(), FUSED),
    # fused, 4-bit: the conv goes native and so does [7, 9] (one-block 4-bit, odd width)
    "adakaon_fused_4bit": (_case("adakaon", lr=1e-3, momentum_dtype="4bit", momentum_4bit_block=8), {1, 3}, FUSED),
    # fused, bf16 params without SR: everything native
    "adakaon_fused_kahan": (_case("adakaon", lr=1e-3, momentum_dtype="int8", bf16_method="kahan"), ALL, FUSED),
    # fused, beta1 = 0: everything native
    "adakaon_fused_nomom": (_case("adakaon", lr=1e-3, betas=(0.0, 0.999), momentum_dtype="int8"), ALL, FUSED),
    "lion": (_case("lion", lr=1e-4, momentum_dtype="bfloat16"), ALL, None),
    "adapnm": (_case("adapnm", lr=1e-3, momentum_dtype="bfloat16"), ALL, None),
    "kprodigy": (_case("kprodigy", lr=1.0, momentum_dtype="bfloat16"), ALL, None),
    "adamuon_gc": (_case("adamuon", lr=2e-2, momentum_dtype="int8", gradient_centralization=True), ALL, None),
    # the removal and the climb ride in the Adakaon apply
    "nekaon_4bit": (_case("nekaon", steps=2, lr=1e-3, momentum_dtype="4bit", momentum_4bit_block=8), ALL, None),
    "nekaon_fused": (_case("nekaon", steps=2, lr=1e-3, momentum_dtype="int8"), {1}, FUSED),
    "msam_global": (_case("msam", steps=2, lr=1e-3, momentum_dtype="int8"), ALL, None),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_grad_after_step(name):
    case, centralized, extra = CASES[name]
    print(f"[gpu] grad writeback {name}", flush=True)
    params = [torch.nn.Parameter(torch.from_numpy(param_values(case, i)).to(DEV, torch.bfloat16))
              for i in range(len(SHAPES))]
    opt = make_opt(case, params, extra=extra)
    for step in range(1, case["steps"] + 1):
        raw = []
        for i, p in enumerate(params):
            p.grad = torch.from_numpy(grad_values(case, i, step)).to(DEV, torch.bfloat16)
            raw.append(to_bits(p.grad))
        opt.step()
    torch.cuda.synchronize()
    for i, p in enumerate(params):
        got = to_bits(p.grad)
        if len(SHAPES[i]) >= 2 and (centralized is ALL or i in centralized):
            want = O.gc_bf16(raw[i].reshape(SHAPES[i][0], -1)).reshape(got.shape)
        else:
            want = raw[i]
        assert np.array_equal(got, want), (name, i, int((got != want).sum()))


def test_fused_big_matrix_keeps_its_grad_and_the_step_is_unchanged():
    """A matrix past the one-block tile (the reference's chunked kernels) keeps its
    p.grad under fused=True; the weights and state equal the fused=False step's."""
    from kaon_amd import Adakaon

    print("[gpu] grad writeback: fused big matrix", flush=True)
    torch.manual_seed(3)
    w = torch.randn(600, 300).to(torch.bfloat16)
    g = (torch.randn(600, 300) * 1e-2).to(torch.bfloat16)
    out = {}
    for fused in (False, True):
        p = torch.nn.Parameter(w.clone().to(DEV))
        p.grad = g.clone().to(DEV)
        opt = Adakaon([p], lr=1e-3, momentum_dtype="int8", fused=fused)
        opt.sr_seed = 9
        opt.step()
        torch.cuda.synchronize()
        out[fused] = (to_bits(p), to_bits(p.grad), to_bits(opt.state[p]["m"]))
    assert np.array_equal(out[True][0], out[False][0])
    assert np.array_equal(out[True][2], out[False][2])
    assert np.array_equal(out[True][1], to_bits(g))
    want = O.gc_bf16(to_bits(g).reshape(600, 300)).reshape(out[False][1].shape)
    assert np.array_equal(out[False][1], want)
