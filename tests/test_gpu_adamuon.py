"""AdaMuon on the GPU against the CPU oracle.

Bit for bit where the step is exact arithmetic: the momentum of the raw
gradient (codes and scales never depend on Newton-Schulz) and the 1-D params
(the Adakaon path with 0.2*lr).  Newton-Schulz is bf16 GEMMs whose fp32
accumulation order differs from the oracle's sequential one, so the
orthogonal factor, the factored state built on it and the weights are compared
within rtol 2e-2, atol 2e-3: the reference's bar for weights stepped by its two
Newton-Schulz paths (tests/test_adamuon.py:154), tighter than its bar for the
orthogonal factor itself (atol 2e-2, tests/test_adamuon.py:109).
"""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

import oracle as O  # noqa: E402
from golden_compare import CASES  # noqa: E402
from gpu_cases import oracle_case_run, run_gpu, to_bits  # noqa: E402

MUON = [k for k, c in CASES.items() if c["opt"] == "adamuon"]


@pytest.fixture(autouse=True, scope="module")
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")


def _state(opt, p):
    return opt.state[p]


@pytest.mark.parametrize("name", MUON)
def test_adamuon_golden_case(name):
    case = CASES[name]
    print(f"[gpu] adamuon case {name}", flush=True)
    oparams, _, _ = oracle_case_run(case)
    params, opt, _ = run_gpu(case)
    for i, (op, p) in enumerate(zip(oparams, params)):
        st = _state(opt, p)
        # momentum: exact
        for k in ("m", "m_scale"):
            if k in op.state:
                gv = to_bits(st[k]).reshape(-1)
                ov = np.asarray(op.state[k]).reshape(-1)
                if gv.dtype != ov.dtype:
                    gv = gv.view(ov.dtype) if gv.itemsize == ov.itemsize else gv.astype(ov.dtype)
                assert int((gv != ov).sum()) == 0, (name, i, k)
        a = O.values(to_bits(p).reshape(op.p.shape), op.p_dtype)
        b = O.values(op.p, op.p_dtype)
        if p.ndim < 2:
            assert np.array_equal(to_bits(p).reshape(-1), op.p.reshape(-1)), (name, i, "1-D weights")
            assert np.array_equal(to_bits(st["v"]).reshape(-1), np.asarray(op.state["v"]).reshape(-1))
        else:
            assert np.allclose(a, b, rtol=2e-2, atol=2e-3), (name, i, np.abs(a - b).max())
            for k in ("row", "col"):
                x, y = st[k].cpu().numpy(), np.asarray(op.state[k])
                assert np.abs(x - y).max() <= 2e-2 * np.abs(y).max() + 1e-30, (name, i, k)


# fp16 params and grads (the reference's per-param path: the momentum of
# grad.float(), subtract_one_ in the param dtype, RN under "stochastic_rounding"
# since the SR write is bf16-only, src/kaon/adamuon.py:565-615,
# src/kaon/_backend.py:82-98).  No reference fixture holds fp16 AdaMuon; the
# oracle's fp16 reads and writes are the ones its fp16 Adakaon goldens pin.
F16_CASES = {
    "adamuon_f16_int8_rn": dict(CASES["adamuon_int8_sr"], p_dtype="f16", g_dtype="f16"),
    "adamuon_f16_bf16_kahan": dict(CASES["adamuon_bf16_rn"], p_dtype="f16", g_dtype="f16",
                                   kwargs=dict(CASES["adamuon_bf16_rn"]["kwargs"], bf16_method="kahan")),
    "adamuon_f16_4bit_none": dict(CASES["adamuon_int8_sr"], p_dtype="f16", g_dtype="f16",
                                  kwargs=dict(CASES["adamuon_int8_sr"]["kwargs"], momentum_dtype="4bit",
                                              bf16_method="none", weight_decay=0.01)),
}


@pytest.mark.parametrize("name", sorted(F16_CASES))
def test_adamuon_fp16_params_match_oracle(name):
    case = F16_CASES[name]
    print(f"[gpu] adamuon fp16 case {name}", flush=True)
    oparams, _, _ = oracle_case_run(case)
    params, opt, _ = run_gpu(case)
    for i, (op, p) in enumerate(zip(oparams, params)):
        assert p.dtype == torch.float16
        st = _state(opt, p)
        for k in ("m", "m_scale"):
            if k in op.state:
                gv = to_bits(st[k]).reshape(-1)
                ov = np.asarray(op.state[k]).reshape(-1)
                if gv.dtype != ov.dtype:
                    gv = gv.view(ov.dtype) if gv.itemsize == ov.itemsize else gv.astype(ov.dtype)
                assert int((gv != ov).sum()) == 0, (name, i, k)
        if p.ndim < 2:
            assert np.array_equal(to_bits(p).reshape(-1), op.p.reshape(-1)), (name, i, "1-D weights")
            if "shift" in op.state:
                assert np.array_equal(to_bits(st["shift"]).reshape(-1), np.asarray(op.state["shift"]).reshape(-1))
        else:
            a = O.values(to_bits(p).reshape(op.p.shape), op.p_dtype)
            b = O.values(op.p, op.p_dtype)
            assert np.allclose(a, b, rtol=2e-2, atol=2e-3), (name, i, np.abs(a - b).max())


def _ns_on_gpu(g: np.ndarray, steps: int) -> np.ndarray:
    """O of one matrix through the phases API (momentum pass with beta1 = 0, so
    M = g; then Newton-Schulz); read back from the plan's workspace."""
    return O.bf16_to_f32(_ns_bits_on_gpu(g, steps)).reshape(g.shape)


def _ns_bits_on_gpu(g: np.ndarray, steps: int) -> np.ndarray:
    """The bf16 bits of O [R, C] (see _ns_on_gpu)."""
    return _ns_bits_many_on_gpu([g], steps)[0]


def _ns_bits_many_on_gpu(gs: list, steps: int) -> list:
    """The bf16 bits of O for several matrices stepped through one plan."""
    return _ns_bits_runs_on_gpu([gs], steps)[0]


def _ns_bits_runs_on_gpu(runs: list, steps: int) -> list:
    """The bf16 bits of O for several matrices, run after run through the same plan and
    workspace, each run with its own gradients (runs[k][i] for matrix i)."""
    from kaon_amd import AdaMuon
    from kaon_amd import _lib as L

    params = []
    for g in runs[0]:
        p = torch.nn.Parameter(torch.zeros(g.shape, dtype=torch.bfloat16, device="cuda"))
        p.grad = torch.from_numpy(g).to("cuda", torch.bfloat16)
        params.append(p)
    opt = AdaMuon(params, betas=(0.0, 0.999), ns_steps=steps)
    group = opt.param_groups[0]
    for p in params:
        opt._init_state(p, opt.state[p], group)
    plan = opt._plan((0, 1, 1, 2), group, params, L.MOM_NONE, {id(p): i for i, p in enumerate(params)},
                     L.OPT_ADAMUON)
    hp = opt._hyper(group, L.BF16, L.BF16)
    s = torch.cuda.current_stream().cuda_stream
    ws16 = plan.workspace.view(torch.int16)
    res = []
    for gs in runs:
        for p, g in zip(params, gs):
            p.grad.copy_(torch.from_numpy(g).to("cuda", torch.bfloat16))
        L.check(L.lib().kaon_adamuon_phases(ctypes.byref(plan.launch), ctypes.byref(hp), (1 << 8) | (1 << 9), s),
                "kaon_adamuon_phases")
        torch.cuda.synchronize()
        out = []
        for i, g in enumerate(gs):
            d = plan.descs[i]
            out.append(ws16[2 * d.ws_aux: 2 * d.ws_aux + g.size].cpu().numpy().view(np.uint16).copy())
        res.append(out)
    return res


def test_newton_schulz_of_a_mixed_plan_equals_each_matrix_alone():
    """Matrices of every tile path in one plan (big and small tiles, transposed, padded 640 -> 768,
    a diagonal-heavy square, enough tiles for the per-XCD lists to interleave tensors and pad with
    idle items): each O is bit for bit the O of that matrix planned alone.  A tile's products do
    not depend on where the planner puts it, so any mix-up of tensors, tiles or idle items shows."""
    print("[gpu] newton-schulz mixed plan", flush=True)
    shapes = [(512, 1024), (1024, 512), (640, 700), (77, 33), (1280, 1280), (130, 300), (768, 1280),
              (5120, 640), (96, 64)]
    rng = np.random.default_rng(11)
    gs = [O.bf16_to_f32(O.f32_to_bf16((rng.standard_normal(s) * 1e-3).astype(np.float32))) for s in shapes]
    together = _ns_bits_many_on_gpu(gs, 2)
    for s, g, o in zip(shapes, gs, together):
        alone = _ns_bits_on_gpu(g, 2)
        assert np.array_equal(o, alone), (s, int((o != alone).sum()))


@pytest.mark.parametrize("shape", [(77, 33), (96, 64), (512, 1024), (1024, 512), (640, 700)])
def test_newton_schulz_nan_gives_torch_nan(shape):
    """A NaN in the gradient makes every element of O NaN, and O holds torch's bf16 NaN
    0x7FC0 (the GEMM epilogues' packed conversion leaves NaN payloads unspecified; the
    last product makes them canonical, in the big-tile kernel only in waves that made one)."""
    print(f"[gpu] newton-schulz NaN {shape}", flush=True)
    rng = np.random.default_rng(7)
    g = O.bf16_to_f32(O.f32_to_bf16((rng.standard_normal(shape) * 1e-3).astype(np.float32)))
    g[shape[0] // 3, shape[1] // 2] = np.nan
    o = _ns_bits_on_gpu(g, 2)
    assert np.all(o == 0x7FC0), np.unique(o)[:8]


def test_newton_schulz_after_a_nan_step_is_clean():
    """A NaN step leaves no trace in the next: with three iterations a product writes the
    iterate's first buffer, padding included (NaN there when the matrix is NaN), and the next
    step's input pass rewrites all of it, padding included, so the clean step's O equals that
    of a fresh plan, bit for bit."""
    print("[gpu] newton-schulz NaN then clean", flush=True)
    shapes = [(640, 700), (130, 300), (1000, 640), (77, 33)]
    rng = np.random.default_rng(5)
    clean = [O.bf16_to_f32(O.f32_to_bf16((rng.standard_normal(s) * 1e-3).astype(np.float32))) for s in shapes]
    bad = [g.copy() for g in clean]
    for g in bad:
        g[g.shape[0] - 1, g.shape[1] - 1] = np.nan
    first, second = _ns_bits_runs_on_gpu([bad, clean], 3)
    fresh = _ns_bits_many_on_gpu(clean, 3)
    for s, o_bad, o, f in zip(shapes, first, second, fresh):
        assert np.all(o_bad == 0x7FC0), s
        assert np.array_equal(o, f), (s, int((o != f).sum()))


# the last six take the 256-tile GEMMs (m = min(R, C) >= 512, padded to a multiple
# of 256 where that grows m^2 by at most 1.5x: 640 -> 768 in the last two):
# symmetric products on row <= column tiles with mirrored stores
@pytest.mark.parametrize("shape", [(64, 96), (96, 64), (77, 33), (130, 300), (256, 640), (640, 256), (320, 2880),
                                   (512, 1024), (1024, 512), (512, 2000), (768, 1280), (640, 700), (1000, 640)])
def test_newton_schulz_matches_oracle(shape):
    print(f"[gpu] newton-schulz {shape}", flush=True)
    rng = np.random.default_rng(sum(shape))
    g = O.bf16_to_f32(O.f32_to_bf16((rng.standard_normal(shape) * 1e-3).astype(np.float32)))
    got = _ns_on_gpu(g, 2)
    want = O.newton_schulz(g, 2)
    assert np.allclose(got, want, rtol=2e-2, atol=2e-3), np.abs(got - want).max()
    # most elements agree to one bf16 rounding step
    close = np.isclose(got, want, rtol=1e-2, atol=1e-4)
    assert close.mean() > 0.95, close.mean()


@pytest.mark.parametrize("shape", [(130, 300), (512, 1024), (1000, 640)])
@pytest.mark.parametrize("steps", [1, 3])
@pytest.mark.parametrize("norm", [None, 4e18])
def test_newton_schulz_steps_and_norms_match_oracle(shape, steps, norm):
    """One step (the first iteration is also the one that writes O) and three (a product writes
    the iterate's first buffer); at an ordinary norm and at ||M|| = 4e18 (squares near the top
    of fp32 in the norm, an undivided product would overflow).  O does not depend on the norm,
    so the bars are the same."""
    print(f"[gpu] newton-schulz {shape} steps={steps} norm={norm}", flush=True)
    rng = np.random.default_rng(sum(shape) + steps)
    sigma = 1e-3 if norm is None else norm / np.sqrt(shape[0] * shape[1])
    g = O.bf16_to_f32(O.f32_to_bf16((rng.standard_normal(shape) * sigma).astype(np.float32)))
    got = _ns_on_gpu(g, steps)
    want = O.newton_schulz(g, steps)
    assert np.all(np.isfinite(got))
    assert np.allclose(got, want, rtol=2e-2, atol=2e-3), np.abs(got - want).max()
    close = np.isclose(got, want, rtol=1e-2, atol=1e-4)
    assert close.mean() > 0.95, close.mean()


def _ns_torch(g: torch.Tensor, steps: int) -> torch.Tensor:
    """zeropower_via_newtonschulz5 (src/kaon/adamuon.py:97-121) restated with torch bf16
    matmuls on the GPU: transpose to the smaller inner dimension, divide by the
    Frobenius norm + 1e-7, then x <- a x + (b A + c A A) x with A = x x^T.  Every
    right-hand operand is made contiguous first."""
    a, b, c = 3.4445, -4.7750, 2.0315
    x = g.bfloat16()
    tr = x.size(0) > x.size(1)
    if tr:
        x = x.t().contiguous()
    x = x / (x.norm() + 1e-7)
    for _ in range(steps):
        aa = torch.matmul(x, x.t().contiguous())
        bb = b * aa + c * torch.matmul(aa, aa.contiguous())
        x = a * x + torch.matmul(bb, x.contiguous())
    if tr:
        x = x.t().contiguous()
    return x.float()


# BASELINE configs[4]'s own matrices: the 1280-row linears and the conv
# [1280, 1280, 3, 3] as 1280 x 11520 (the 256-tile GEMM path), [5120, 1280]
# transposed, and a 640-row conv (256 tiles over rows padded to 768)
@pytest.mark.parametrize("shape", [(1280, 1280), (1280, 2048), (1280, 5120), (5120, 1280), (1280, 11520),
                                   (640, 5760)])
def test_newton_schulz_sdxl_sizes_match_torch(shape):
    """Newton-Schulz at the SDXL set's sizes (too large for the scalar oracle) against
    the reference's iteration run with torch's bf16 GEMMs on the same device: within
    rtol 2e-2, atol 2e-3 (the module's bar), most elements within one bf16 step."""
    print(f"[gpu] newton-schulz sdxl {shape}", flush=True)
    rng = np.random.default_rng(sum(shape) + 1)
    g = O.bf16_to_f32(O.f32_to_bf16((rng.standard_normal(shape) * 1e-3).astype(np.float32)))
    got = _ns_on_gpu(g, 2)
    want = _ns_torch(torch.from_numpy(g).cuda(), 2).cpu().numpy()
    assert np.allclose(got, want, rtol=2e-2, atol=2e-3), np.abs(got - want).max()
    close = np.isclose(got, want, rtol=1e-2, atol=1e-4)
    assert close.mean() > 0.95, close.mean()


def test_newton_schulz_orthogonalizes():
    """Five quintic steps leave every singular value in (0.5, 1.3)."""
    rng = np.random.default_rng(7)
    g = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((128, 512)).astype(np.float32)))
    o = _ns_on_gpu(g, 5)
    sv = np.linalg.svd(o.astype(np.float64), compute_uv=False)
    assert sv.min() > 0.5 and sv.max() < 1.3, (sv.min(), sv.max())


@pytest.mark.parametrize("md,wd", [("int8", 0.0), ("int8", 0.01), ("4bit", 0.0)])
def test_specialized_apply_matches_generic_kernel(md, wd):
    """The keep count and apply on the specialized row-set kernel (bf16 p and g, SR,
    C % 8 == 0) against the generic kernel on the same inputs: two optimizers over
    identical params and grads, the second with its plans' fast slices handed to
    the generic kernel (KaonLaunch.n_fast = 0).  Newton-Schulz runs the same
    kernels on the same bytes in both, so weights, codes and scales must agree
    bit for bit."""
    from kaon_amd import AdaMuon

    print(f"[gpu] adamuon fast vs generic apply {md} wd={wd}", flush=True)
    shapes = [(320, 1280), (256, 256, 3, 3), (640, 640)]
    gen = torch.Generator(device="cpu").manual_seed(5)
    init = [(torch.randn(*s, generator=gen) * 0.02).bfloat16() for s in shapes]
    grads = [[(torch.randn(*s, generator=gen) * 1e-3).bfloat16() for s in shapes] for _ in range(3)]
    kw = dict(lr=2e-2, betas=(0.95, 0.999), momentum_dtype=md, ns_steps=2, weight_decay=wd)
    runs = []
    for generic in (False, True):
        params = [torch.nn.Parameter(t.clone().cuda()) for t in init]
        opt = AdaMuon(params, **kw)
        opt.sr_seed = 17
        for step, gs in enumerate(grads):
            # grads copied into the same tensors, so the cached plans stay in use
            for p, g in zip(params, gs):
                if p.grad is None:
                    p.grad = g.clone().cuda()
                else:
                    p.grad.copy_(g)
            if generic and step == 1:
                for _key, (_ptrs, plan) in opt._plans.items():
                    assert plan.launch.n_fast > 0
                    plan.launch.n_fast = 0
            opt.step()
        if generic:
            assert all(plan.launch.n_fast == 0 for _k, (_p, plan) in opt._plans.items())
        torch.cuda.synchronize()
        runs.append((params, opt))
    (pa, oa), (pb, ob) = runs
    for i, (a, b) in enumerate(zip(pa, pb)):
        assert np.array_equal(to_bits(a), to_bits(b)), (md, i, "weights")
        for k in ("m", "m_scale"):
            assert np.array_equal(to_bits(oa.state[a][k]).reshape(-1), to_bits(ob.state[b][k]).reshape(-1)), (md, i, k)
