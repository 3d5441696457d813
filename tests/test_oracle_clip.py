"""Pin the RMS clip's sum of squares against a float64 computation of its definition.

The clip divides the update U by max(rms(U) / clip_threshold, 1), rms(U) =
sqrt(sum U^2 / n) (src/kaon/adakaon.py:1000-1002, src/kaon/_factored.py:84-89),
with U = (G * r) * c, r = rsqrt(row / mean(row)), c = rsqrt(col) for a factored
tensor and U = g * rsqrt(v) for a 1-D one.  The oracle forms the sum three ways:

* canonical Adakaon / AdaMuon: the algebraic form rm * sum_j (1 / col_j)
  sum_i G_ij^2 / row_i, built from column partials during the row EMA;
* torch order: torch CPU's sum of the squares of U itself;
* AdaPNM: the canonical per-row sums of U^2.

Each is checked against sum U^2 computed in float64 from the oracle's own state
after the step (the new row / col / v) and the centralized gradient, at steps
1-3 (where the new row differs from the old one by a factor of 1.3-2), over
tensors with all-zero gradient rows (which add nothing to sum U^2 but would add
eps1 / row_i per element to a sum built from the eps1-carrying squares), more
than one 2048-column finalize item, ragged rows and a 1-D tensor.
"""
import numpy as np
import pytest

import oracle as O
from golden_compare import group_for

SHAPES = [[300, 72], [40, 1280], [64, 2500], [6, 3, 3, 3], [1000]]
ZERO_ROWS = {0: range(5, 21), 2: range(0, 10)}
TOL = 1e-5  # fp32 sums of <= 160,000 terms in trees and short sequential runs


def _grads(step, rng_seed=7):
    rng = np.random.default_rng(rng_seed * 1000 + step)
    out = []
    for i, shape in enumerate(SHAPES):
        R = shape[0]
        g = rng.standard_normal(shape).astype(np.float32)
        scale = np.exp(rng.uniform(-6, 1, size=(R,) + (1,) * (len(shape) - 1))).astype(np.float32)
        g = g * (scale if len(shape) > 1 else np.float32(0.3))
        for r in ZERO_ROWS.get(i, ()):
            g[r] = 0.0
        out.append(g)
    return out


def _ss64(prm, g_bits):
    """sum U^2 in float64 from the state after the step."""
    R, C = prm.eff
    if prm.factored:
        G = O.bf16_to_f32(O.gc_bf16(g_bits.reshape(R, C))).astype(np.float64)
        row = prm.state["row"].astype(np.float64)
        col = prm.state["col"].astype(np.float64)
        r = 1.0 / np.sqrt(row / row.mean())
        U = G * r[:, None] * (1.0 / np.sqrt(col))[None, :]
    else:
        g = O.bf16_to_f32(g_bits.reshape(-1)).astype(np.float64)
        U = g / np.sqrt(prm.state["v"].astype(np.float64))
    return float((U * U).sum())


def _run(torch_order):
    """Three Adakaon steps; each step's clip sums against float64."""
    case = dict(opt="adakaon", kwargs=dict(lr=1e-3, betas=(0.9, 0.999), momentum_dtype="float32",
                                           clip_threshold=0.5))
    rng = np.random.default_rng(3)
    params = [O.make_param(s, O.BF16, O.BF16, tensor_id=i, p_values=rng.standard_normal(s).astype(np.float32))
              for i, s in enumerate(SHAPES)]
    opt = O.OracleOptimizer(params, "adakaon", group_for(case), seed=11)
    for step in (1, 2, 3):
        for prm, g in zip(params, _grads(step)):
            prm.g = O.f32_to_bf16(g).reshape(prm.shape)
        ss = {i: np.zeros(1, np.float32) for i in range(len(SHAPES))}
        if torch_order:
            with O.torch_order():
                opt.step(ss_out=ss)
        else:
            opt.step(ss_out=ss)
        for i, prm in enumerate(params):
            want = _ss64(prm, prm.g)
            got = float(ss[i][0])
            rel = abs(got - want) / want
            assert rel <= TOL, (torch_order, step, i, got, want, rel)
    return params


@pytest.mark.parametrize("torch_order", [False, True], ids=["canonical", "torch"])
def test_adakaon_clip_sum_of_squares_is_sum_u2(torch_order):
    _run(torch_order)


def test_zero_rows_add_nothing():
    """The same step with the zero rows' squares counted (eps1 carried into the
    algebraic sum) would be far off: the zero rows alone would contribute about as
    much as the others.  Shown here by the float64 sum of eps1 / row_i / col_j * rm
    over those rows being a large fraction of sum U^2, so a sum that included it
    could not pass the 1e-5 check above."""
    params = _run(False)
    prm = params[0]
    R, C = prm.eff
    row = prm.state["row"].astype(np.float64)
    col = prm.state["col"].astype(np.float64)
    rm = row.mean()
    zr = np.array(list(ZERO_ROWS[0]))
    extra = 1e-30 * rm * (1.0 / row[zr]).sum() * (1.0 / col).sum()
    assert extra / _ss64(prm, prm.g) > 0.01


def test_adapnm_clip_sum_is_reported():
    """AdaPNM keeps the per-row canonical form; the diagnostics output is written."""
    case = dict(opt="adapnm", kwargs=dict(lr=1e-3, momentum_dtype="float32", clip_threshold=0.5))
    rng = np.random.default_rng(5)
    params = [O.make_param(s, O.BF16, O.BF16, tensor_id=i, p_values=rng.standard_normal(s).astype(np.float32))
              for i, s in enumerate(SHAPES)]
    opt = O.OracleOptimizer(params, "adapnm", group_for(case), seed=11)
    for prm, g in zip(params, _grads(1)):
        prm.g = O.f32_to_bf16(g).reshape(prm.shape)
    ss = {i: np.full(1, -1.0, np.float32) for i in range(len(SHAPES))}
    opt.step(ss_out=ss)
    assert all(np.isfinite(v[0]) and v[0] > 0 for v in ss.values())
