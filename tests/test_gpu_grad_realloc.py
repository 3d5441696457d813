"""Gradient storage that moves between steps (the caching allocator's pattern when a
new input shape's backward runs): the step must read every param's current .grad.

Step 1 takes fresh gradients.  Before step 2, param 0's gradient is refilled in place
(same storage, new values) and params 1-3 get new gradient tensors while their old
buffers are overwritten with NaN, standing in for freed memory the allocator hands out
again.  The cached plan must be rebuilt from the new storage pointers: the weights and
state after step 2 equal the oracle's bit for bit (the oracle never sees the poison).
A second run refills every gradient in place, so the plan is reused."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

from cases import grad_values, param_values  # noqa: E402
from gpu_cases import DEV, assert_same_as_oracle, make_opt, oracle_case_run  # noqa: E402


@pytest.fixture(autouse=True, scope="module")
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")


def _case(opt, kwargs):
    return dict(steps=2, seed=5, p_dtype="bf16", g_dtype="bf16", opt=opt, shapes=[[64, 48], [64, 48], [40, 20], [1280]],
                kwargs=kwargs)


CASES = {
    "adakaon_int8": _case("adakaon", dict(lr=1e-3, betas=(0.6, 0.999), momentum_dtype="int8")),
    "nekaon_4bit_b64": _case("nekaon", dict(lr=1e-4, k=1.5, momentum_dtype="4bit", momentum_4bit_block=64)),
    "lion_int8": _case("lion", dict(lr=2e-4, betas=(0.95, 0.98), momentum_dtype="int8")),
}


def _grad(case, i, step):
    return torch.from_numpy(grad_values(case, i, step)).to(DEV, torch.bfloat16)


@pytest.mark.parametrize("moved", [True, False], ids=["moved", "in_place"])
@pytest.mark.parametrize("name", sorted(CASES))
def test_step_reads_the_current_grad_storage(name, moved):
    case = CASES[name]
    print(f"[gpu] grad storage {name} moved={moved}", flush=True)
    params = [torch.nn.Parameter(torch.from_numpy(np.ascontiguousarray(param_values(case, i))).to(DEV, torch.bfloat16))
              for i in range(len(case["shapes"]))]
    opt = make_opt(case, params)
    old = [_grad(case, i, 1) for i in range(len(params))]
    for p, g in zip(params, old):
        p.grad = g
    opt.step()
    for i, p in enumerate(params):
        g2 = _grad(case, i, 2)
        if moved and i > 0:
            p.grad = g2.clone()           # new storage
            old[i].fill_(float("nan"))    # the old storage, poisoned
        else:
            p.grad.copy_(g2)              # same storage, new values
    opt.step()
    torch.cuda.synchronize()
    oparams, _, _ = oracle_case_run(case)
    assert_same_as_oracle(case, oparams, params, opt, label=f"{name} moved={moved}")
