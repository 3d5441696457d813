"""Pin the oracle's rounding model against torch CPU (the reference's arithmetic).

The reference computes its step with torch ops; torch is a dependency of the
reference (pyproject: torch>=2.5), importable here, so its CPU kernels are
the ground truth for one-op rounding questions the fixtures cannot isolate:

* lerp(a, b, w) with a python-float weight: both branches of |w| < 0.5 and the
  fused multiply-add in each (src/kaon/_factored.py:51-52,
  src/kaon/_momentum_codec.py:268, 305, 367);
* bf16 <-> fp32 conversion, round to nearest even (every bf16 store);
* GC in the grad dtype: bf16 row mean, bf16 subtraction
  (src/kaon/_backend.py:147-177) on rows short enough that torch's fp32 sum
  is exact, so the reduction order cannot matter;
* the SR bit trick against its three-op torch form
  (src/kaon/_stochastic_rounding.py:88-103);
* addcmul_(g, g, value=s) after mul_(beta2): AdaPNM's 1-D second moment
  (src/kaon/adapnm.py:1243-1244), one fma of (s * g) and g into v * beta2;
* add_(x, alpha) on bf16 tensors: KProdigy's bf16 momentum
  (src/kaon/kprodigy.py:738-740) -- torch CPU's vector loop rounds alpha to bf16.

* the fp32 reduction orders of the five sums in a step (the oracle's
  torch-order mode, KoTensor.torch_order): x.sum() / x.mean(-1) of a contiguous
  row, x.mean(-2) over the rows, the bf16 GC mean, and t.norm(2) -- each
  reproduced bit for bit (ko_torch_inner_sum, ko_torch_outer_sum,
  ko_torch_sumsq) on sizes that cross every cascade level and vector tail.

A plausible slip -- a lerp without the fma, the branch threshold on the wrong
side, truncation instead of RNE, an fp32 instead of a bf16 GC, a 16-lane
instead of an 8-lane norm, a cascade level too few -- fails one of these on the
seeded inputs.
"""
import numpy as np
import pytest
import torch

import oracle as O


@pytest.mark.parametrize("w", [0.1, 0.001, 0.4999, 0.5, 0.75, 0.999, 1e-30, -0.3, 1.0])
def test_lerp_matches_torch_cpu(w):
    rng = np.random.default_rng(1)
    a = (rng.standard_normal(200_000) * np.exp(rng.uniform(-20, 20, 200_000))).astype(np.float32)
    b = (rng.standard_normal(200_000) * np.exp(rng.uniform(-20, 20, 200_000))).astype(np.float32)
    b[:1000] = a[:1000] * np.float32(1.0000001)  # nearly equal operands: cancellation in b - a
    want = torch.from_numpy(a.copy()).lerp_(torch.from_numpy(b), w).numpy()
    got = O.lerp(a, b, w)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_lerp_fma_is_observable():
    """Inputs on which an unfused lerp differs from the fused one (so the test
    above really pins the fma, not just the formula)."""
    rng = np.random.default_rng(2)
    a = rng.standard_normal(100_000).astype(np.float32)
    b = rng.standard_normal(100_000).astype(np.float32)
    w = np.float32(0.1)
    unfused = (a + w * (b - a)).astype(np.float32)
    fused = O.lerp(a, b, float(w))
    assert (unfused.view(np.uint32) != fused.view(np.uint32)).sum() > 100


def test_bf16_conversion_matches_torch():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(300_000) * np.exp(rng.uniform(-80, 80, 300_000))).astype(np.float32)
    x[:4] = [np.inf, -np.inf, 3.3961e38, -0.0]
    # exact ties at every mantissa parity
    ties = (np.arange(1, 2000, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    x = np.concatenate([x, ties])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.f32_to_bf16(x), want)


@pytest.mark.parametrize("shape", [(7, 16), (33, 40), (5, 128)])
def test_gc_bf16_matches_torch_on_exact_sum_rows(shape):
    """Rows of <= 128 bf16 values with a shared exponent range sum exactly in
    fp32 in any order, so torch's result is order-free and must equal the oracle's."""
    rng = np.random.default_rng(4)
    g = torch.from_numpy((rng.integers(-255, 256, shape) / 256.0).astype(np.float32)).to(torch.bfloat16)
    want = g - g.mean(dim=1, keepdim=True)
    got = O.gc_bf16(g.view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(got, want.view(torch.int16).numpy().view(np.uint16))


def test_sr_round_matches_three_op_torch_form():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(100_000) * np.exp(rng.uniform(-30, 30, 100_000))).astype(np.float32)
    noise = rng.integers(0, 1 << 16, x.size).astype(np.uint16)
    t = torch.from_numpy(x.copy()).view(torch.int32)
    t.add_(torch.from_numpy(noise.astype(np.int32))).bitwise_and_(-65536)
    want = t.view(torch.float32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.sr_round(x, noise), want)


def test_pnm_addcmul_second_moment_matches_torch():
    """The oracle's AdaPNM 1-D ``v`` after three steps equals torch CPU's
    ``v.mul_(beta2).addcmul_(g, g, value=1 - beta2)`` bit for bit; the unfused
    form (two products and an add) differs on these inputs, so the fma is pinned."""
    from golden_compare import DEFAULTS

    n, b2 = 4096, 0.99
    group = dict(DEFAULTS["adapnm"], betas=(0.8, b2), momentum_dtype="float32")
    rng = np.random.default_rng(7)
    prm = O.make_param((n,), O.F32, O.F32, p_values=np.zeros(n, dtype=np.float32))
    opt = O.OracleOptimizer([prm], "adapnm", group)
    v = torch.zeros(n)
    unfused = np.zeros(n, dtype=np.float32)
    fb2, fa2 = np.float32(b2), np.float32(1.0 - b2)
    for _ in range(3):
        g = (rng.standard_normal(n) * np.exp(rng.uniform(-6, 0, n))).astype(np.float32)
        prm.g = g.copy()
        opt.step()
        v.mul_(b2).addcmul_(torch.from_numpy(g), torch.from_numpy(g), value=1.0 - b2)
        unfused = (unfused * fb2 + ((fa2 * g) * g).astype(np.float32)).astype(np.float32)
    want = v.numpy()
    assert np.array_equal(prm.state["v"].view(np.uint32), want.view(np.uint32))
    assert (unfused.view(np.uint32) != want.view(np.uint32)).sum() > 10


def test_bf16_add_alpha_is_rounded_to_bf16_by_torch_cpu():
    """KProdigy's bf16 momentum is m.mul_(beta1).add_(g.to(bf16), alpha=d*(1-beta1))
    (kprodigy.py:738-740).  torch CPU's 32-wide vector loop rounds alpha to bf16
    (an fp32 alpha differs on most elements; the oracle's KProdigy pass 1 uses the
    bf16 one).  On a length that is a multiple of 32 (no scalar tail) the bf16-alpha
    form matches every element; the fp32-alpha form does not."""
    torch.set_num_threads(1)
    rng = np.random.default_rng(9)
    n = 32 * 4096
    g = torch.from_numpy((rng.standard_normal(n) * 1e-3).astype(np.float32)).bfloat16()
    m0 = torch.from_numpy((rng.standard_normal(n) * 1e-9).astype(np.float32)).bfloat16()
    alpha, b1 = 3.3e-5 * 0.1, 0.9
    want = m0.clone().mul_(b1).add_(g, alpha=alpha).float().numpy()
    mb = O.bf16_to_f32(O.f32_to_bf16(O.bf16_to_f32(O.f32_to_bf16(m0.float().numpy())) * np.float32(b1)))
    gf = g.float().numpy()
    ab = O.bf16_to_f32(O.f32_to_bf16(np.array([alpha], dtype=np.float32)))[0]
    exact = mb.astype(np.float64) + np.float64(ab) * gf.astype(np.float64)  # exact product of two bf16
    got = O.bf16_to_f32(O.f32_to_bf16(exact.astype(np.float32)))
    assert np.array_equal(got, want)
    f32a = O.bf16_to_f32(O.f32_to_bf16((mb + np.float32(alpha) * gf).astype(np.float32)))
    assert (f32a != want).sum() > n // 10


_SIZES = [1, 7, 8, 9, 31, 32, 33, 64, 100, 255, 256, 257, 640, 1280, 2048, 2880, 4097, 5760, 11520, 65536 + 17,
          300_000]


def test_torch_row_sum_order_reproduced():
    """torch CPU's fp32 x.sum() and row sums (the inner cascade with 8-float vectors)."""
    torch.set_num_threads(1)
    rng = np.random.default_rng(21)
    for n in _SIZES:
        x = (rng.standard_normal(n) * np.exp(rng.uniform(-8, 8, n))).astype(np.float32)
        want = np.float32(torch.from_numpy(x).sum().item())
        assert O.torch_inner_sum(x).view(np.uint32) == want.view(np.uint32), n
    for C in (1280, 5, 3):
        x = (rng.standard_normal((37, C)) ** 2 * 1e-6).astype(np.float32)
        want = torch.from_numpy(x).mean(dim=-1).numpy()
        got = np.array([O.torch_inner_sum(r) for r in x], np.float32) / np.float32(C)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), C


@pytest.mark.parametrize("shape", [(320, 2880), (1280, 1280), (17, 40), (640, 5760), (100, 13), (5, 300), (9, 1),
                                   (33, 6), (70, 4), (3, 7)])
def test_torch_column_sum_order_reproduced(shape):
    """torch CPU's x.mean(dim=-2) of an fp32 matrix (the outer cascade: 32-column blocks,
    then 8-column blocks and single columns through the 4-way row split)."""
    torch.set_num_threads(1)
    rng = np.random.default_rng(22)
    x = (rng.standard_normal(shape) ** 2 * np.exp(rng.uniform(-6, 6, shape))).astype(np.float32)
    want = torch.from_numpy(x).mean(dim=-2).numpy()
    got = O.torch_outer_sum(x) / np.float32(shape[0])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_torch_norm_order_reproduced():
    """torch CPU's fp32 t.norm(2): 8 lanes of sequential fused multiply-adds, lanes
    added in order, then the tail.  A 16-lane model or an unfused one fails."""
    torch.set_num_threads(1)
    rng = np.random.default_rng(23)
    for n in _SIZES:
        x = (rng.standard_normal(n) * np.exp(rng.uniform(-6, 6, n))).astype(np.float32)
        want = np.float32(torch.from_numpy(x).norm(2).item())
        got = np.sqrt(O.torch_sumsq(x), dtype=np.float32)
        assert got.view(np.uint32) == want.view(np.uint32), n


def test_torch_bf16_mean_is_one_rounding_of_the_fp32_cascade_sum():
    """g.mean(dims) on bf16: the bf16 rounding of (fp32 cascade sum of the upcast row) / C."""
    torch.set_num_threads(1)
    rng = np.random.default_rng(24)
    for C in (640, 1280, 2048, 2880, 5760):
        g = torch.from_numpy((rng.standard_normal((200, C)) * np.exp(rng.uniform(-4, 4, (200, 1))))
                             .astype(np.float32)).bfloat16()
        want = g.mean(dim=1).view(torch.int16).numpy().view(np.uint16)
        sums = np.array([O.torch_inner_sum(r) for r in g.float().numpy()], np.float32)
        assert np.array_equal(O.f32_to_bf16(sums / np.float32(C)), want), C
