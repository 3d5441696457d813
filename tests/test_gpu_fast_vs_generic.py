"""The specialized phase-5/6 kernel against the generic one at SDXL sizes.

The oracle pins both kernels on small and mid-sized cases (tests/test_gpu_*.py).
At the SDXL set's own sizes the oracle is slow, so here the two kernels pin
each other: two optimizers step identical params with identical grads, the
second with its plans' fast slices handed to the generic kernel
(KaonLaunch.n_fast = 0, which the C ABI documents as result-preserving).
Weights, momentum codes and scales and the factored state must agree bit for
bit after every step, for each optimizer and codec the specialized kernel takes.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

from gpu_cases import to_bits  # noqa: E402

SHAPES = [(1280, 1280, 3, 3), (5120, 1280), (640, 640, 3, 3), (1280, 640)]


@pytest.fixture(autouse=True, scope="module")
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")


def _make(name, params):
    import kaon_amd as K

    if name == "adakaon_int8":
        return K.Adakaon(params, lr=1e-4, momentum_dtype="int8")
    if name == "adakaon_4bit_b128_wd":
        return K.Adakaon(params, lr=1e-4, momentum_dtype="4bit", momentum_4bit_block=128, weight_decay=0.01)
    if name == "lion_int8":
        return K.Lion(params, lr=2e-4, betas=(0.95, 0.98), momentum_dtype="int8")
    if name == "nekaon_4bit_b256":
        return K.Nekaon(params, lr=1e-4, betas=(0.2, 0.999), momentum_dtype="4bit", momentum_4bit_block=256)
    if name == "adapnm_bf16":
        return K.AdaPNM(params, lr=1e-4, momentum_dtype="bfloat16")
    raise ValueError(name)


@pytest.mark.parametrize("name", ["adakaon_int8", "adakaon_4bit_b128_wd", "lion_int8", "nekaon_4bit_b256",
                                  "adapnm_bf16"])
def test_specialized_kernel_matches_generic_at_sdxl_sizes(name):
    print(f"[gpu] fast vs generic {name}", flush=True)
    gen = torch.Generator(device="cpu").manual_seed(11)
    init = [(torch.randn(*s, generator=gen) * 0.02).bfloat16() for s in SHAPES]
    grads = [[(torch.randn(*s, generator=gen) * 10.0 ** (-3 - i)).bfloat16() for i, s in enumerate(SHAPES)]
             for _ in range(3)]
    runs = []
    for generic in (False, True):
        params = [torch.nn.Parameter(t.clone().cuda()) for t in init]
        opt = _make(name, params)
        inner = getattr(opt, "inner", opt)
        inner.sr_seed = 23
        for step, gs in enumerate(grads):
            for p, g in zip(params, gs):
                if p.grad is None:
                    p.grad = g.clone().cuda()
                else:
                    p.grad.copy_(g)
            if generic and step == 1:
                assert any(plan.launch.n_fast > 0 for _k, (_p, plan) in inner._plans.items())
                for _k, (_p, plan) in inner._plans.items():
                    plan.launch.n_fast = 0
            opt.step()
        if generic:
            assert all(plan.launch.n_fast == 0 for _k, (_p, plan) in inner._plans.items())
        torch.cuda.synchronize()
        runs.append((params, inner))
    (pa, ia), (pb, ib) = runs
    for i, (a, b) in enumerate(zip(pa, pb)):
        assert np.array_equal(to_bits(a), to_bits(b)), (name, i, "weights")
        sa, sb = ia.state[a], ib.state[b]
        assert sorted(sa) == sorted(sb)
        for k in sa:
            if torch.is_tensor(sa[k]):
                assert np.array_equal(to_bits(sa[k]).reshape(-1), to_bits(sb[k]).reshape(-1)), (name, i, k)
