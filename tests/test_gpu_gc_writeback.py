"""p.grad after a step with gradient centralization.

The reference's native paths (Adakaon / AdaPNM with fused=False, and Lion,
AdaMuon, KProdigy, which have no fused path) centralize p.grad in place
before stepping (centralize_grads_, src/kaon/_backend.py:147-177), so a
caller reading p.grad after step() sees g - mean over the fan-in, in the
grad dtype, for params of 2 dims or more.  The fused Adakaon / AdaPNM kernels
centralize in-kernel and leave p.grad as it was (src/kaon/adakaon.py:387-409).
The Adakaon / Lion apply and KProdigy's pass 2 store the centralized gradient
as they read it (KAON_F_GC_WRITE); AdaPNM and AdaMuon write it back after the
step with kaon_gc_writeback.  Checked against the oracle's bf16 GC.
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


def _case(opt, **kw):
    return dict(steps=1, seed=5, p_dtype="bf16", g_dtype="bf16", opt=opt, shapes=SHAPES, kwargs=kw)


CASES = {
    "adakaon_native": (_case("adakaon", lr=1e-3, momentum_dtype="int8"), True),
    "adakaon_fused": (_case("adakaon", lr=1e-3, momentum_dtype="int8"), False),
    "lion": (_case("lion", lr=1e-4, momentum_dtype="bfloat16"), True),
    "adapnm": (_case("adapnm", lr=1e-3, momentum_dtype="bfloat16"), True),
    "kprodigy": (_case("kprodigy", lr=1.0, momentum_dtype="bfloat16"), True),
    "adamuon_gc": (_case("adamuon", lr=2e-2, momentum_dtype="int8", gradient_centralization=True), True),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_grad_after_step(name):
    case, centralized = CASES[name]
    print(f"[gpu] grad writeback {name}", flush=True)
    params = [torch.nn.Parameter(torch.from_numpy(param_values(case, i)).to(DEV, torch.bfloat16))
              for i in range(len(SHAPES))]
    opt = make_opt(case, params)
    if name == "adakaon_fused":
        opt.centralize_grads_in_place = False  # what Adakaon(fused=True) sets
    raw = []
    for i, p in enumerate(params):
        p.grad = torch.from_numpy(grad_values(case, i, 1)).to(DEV, torch.bfloat16)
        raw.append(to_bits(p.grad))
    opt.step()
    torch.cuda.synchronize()
    for i, p in enumerate(params):
        got = to_bits(p.grad)
        if len(SHAPES[i]) >= 2 and centralized:
            want = O.gc_bf16(raw[i].reshape(SHAPES[i][0], -1)).reshape(got.shape)
        else:
            want = raw[i]
        assert np.array_equal(got, want), (name, i, int((got != want).sum()))


def test_fused_adakaon_leaves_grad_and_native_writes_it():
    from kaon_amd import Adakaon

    p = [torch.nn.Parameter(torch.zeros(8, 16, device=DEV))]
    assert Adakaon(p).centralize_grads_in_place
    assert not Adakaon(p, fused=True).centralize_grads_in_place
