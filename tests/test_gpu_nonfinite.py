"""GPU parity with non-finite and degenerate gradients: NaN, +inf and -inf written
into p.grad, and all-zero rows, on the steps the case names (the faults a host-side
test can force on the reference's step).  The HIP step against the CPU oracle: bf16
weights and momentum codes bit for bit; fp32 values (weights, scales, the factored /
1-D state) bit for bit where they are numbers and NaN at the same places (a NaN's
payload is not compared: the device's invalid operations give the canonical
0x7FC00000, the x86 host's 0xFFC00000)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

import oracle as O  # noqa: E402
from gpu_cases import oracle_case_run, run_gpu, state_of, to_bits  # noqa: E402


@pytest.fixture(autouse=True, scope="module")
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")


def _same(got, want, what):
    got = np.asarray(got).reshape(-1)
    want = np.asarray(want).reshape(-1)
    if got.dtype != want.dtype:
        got = got.view(want.dtype) if got.itemsize == want.itemsize else got.astype(want.dtype)
    if want.dtype.kind == "f":
        gn, wn = np.isnan(got), np.isnan(want)
        assert np.array_equal(gn, wn), f"{what}: NaN at {int((gn != wn).sum())} other places"
        g, w = got[~gn], want[~wn]
        bad = int((g.view(np.uint32 if g.itemsize == 4 else np.uint16) !=
                   w.view(np.uint32 if w.itemsize == 4 else np.uint16)).sum())
    else:
        bad = int((got != want).sum())
    assert bad == 0, f"{what}: {bad}/{got.size} differ"


def _check(case, oparams, params, opt, label):
    for i, (op, p) in enumerate(zip(oparams, params)):
        bits = to_bits(p).reshape(-1)
        want = op.p.reshape(-1)
        if bits.dtype == np.float32:
            _same(bits, want, f"{label} param {i} weights")
        else:
            assert int((bits != want).sum()) == 0, f"{label} param {i}: {int((bits != want).sum())} weights differ"
        st = state_of(opt, p)
        for k, ov in op.state.items():
            if k.startswith("_") or k.endswith("_numel") or k.endswith("_block") or k == "step":
                continue
            _same(to_bits(st[k]), ov, f"{label} param {i} state {k}")


def _case(opt, kwargs, steps=3, p="bf16", g="bf16", **kw):
    # short packed rows, a one-row vector, a conv, a fast-path matrix, a ragged matrix
    shapes = [[64, 96], [40, 20], [1280], [3, 5, 7], [2, 5120], [7, 129]]
    poison = {1: [(0, "nan", 5), (1, "inf", 17), (2, "-inf", 3), (5, "zero_row", 2)],
              2: [(3, "zero_row", 1), (4, "nan", 5000), (5, "inf", 100), (0, "-inf", 700)]}
    c = dict(steps=steps, seed=11, p_dtype=p, g_dtype=g, opt=opt, shapes=shapes, kwargs=kwargs, poison=poison)
    c.update(kw)
    return c


CASES = {
    "ada_int8": _case("adakaon", dict(lr=1e-3, betas=(0.9, 0.999), momentum_dtype="int8", weight_decay=0.05)),
    "ada_4bit_b64_clip": _case("adakaon", dict(lr=1e-3, momentum_dtype="4bit", momentum_4bit_block=64,
                                               clip_threshold=0.05)),
    "ada_bf16_f32": _case("adakaon", dict(lr=1e-3, momentum_dtype="bfloat16", weight_decay=0.1), p="f32", g="f32"),
    "lion_int8": _case("lion", dict(lr=2e-4, betas=(0.95, 0.98), momentum_dtype="int8", weight_decay=0.1)),
    "nekaon_int8": _case("nekaon", dict(lr=1e-4, k=1.5, momentum_dtype="int8"), steps=4),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_nonfinite_grads_match_oracle(name):
    case = CASES[name]
    print(f"[gpu] non-finite grads {name}", flush=True)
    oparams, _, _ = oracle_case_run(case)
    params, opt, _ = run_gpu(case)
    _check(case, oparams, params, opt, name)


TORCH_CASES = ("ada_int8", "ada_bf16_f32", "lion_int8", "nekaon_int8")


@pytest.mark.parametrize("name", TORCH_CASES)
def test_nonfinite_grads_match_oracle_in_torch_order(name):
    """The same poisoned gradients through the torch-order kernels (reduction_order="torch":
    torch CPU's cascades for the means, its 8 fma chains for the clip norm), against the
    oracle in that order."""
    case = CASES[name]
    print(f"[gpu] non-finite grads, torch order {name}", flush=True)
    with O.torch_order():
        oparams, _, _ = oracle_case_run(case)
    params, opt, _ = run_gpu(case, extra={"reduction_order": "torch"})
    _check(case, oparams, params, opt, f"{name} torch order")
