"""kaon_adakaon_step_noalloc (static device workspace) against kaon_adakaon_step.

Two optimizers step identical copies of the same params and grads: one
through kaon_adakaon_step with its plan's workspace, the other through the
allocation-free entry point, which takes the workspace from the library's
static device array.  Weights and every state tensor must agree bit for bit,
on two calls in a row (the second plan smaller than the first, so the array
still holds the first call's contents), over two steps each.  A plan larger
than the static workspace is refused with an error, before any launch.  In torch
order the allocation-free step keeps the long clip chains on the caller's stream
(no side stream) and agrees with the two-stream step.
"""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.fixture(autouse=True, scope="module")
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")


def _noalloc_fn():
    from kaon_amd import _lib as L

    return L.lib().kaon_adakaon_step_noalloc


def _bits(t):
    t = t.detach().contiguous().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy()
    return t.numpy()


def _step_noalloc(opt):
    """One Adakaon step of ``opt`` through kaon_adakaon_step_noalloc."""
    from kaon_amd import _engine as E
    from kaon_amd import _lib as L

    fn = _noalloc_fn()
    opt._t += 1
    for gid, group in enumerate(opt.param_groups):
        params, pkey = opt._stepped(group)
        for plan, pdt, gdt, dev in opt._launches(gid, group, params, pkey):
            hp = opt._hyper(group, pdt, gdt, None, gid)
            assert plan.launch.ws_words == plan.info.ws_words
            rc = fn(ctypes.byref(plan.launch), ctypes.byref(hp), E.stream_handle(dev))
            L.check(rc, "kaon_adakaon_step_noalloc")


def _run(shapes, momentum_dtype, seed, steps=2, **kw):
    from kaon_amd import Adakaon

    rng = np.random.default_rng(seed)
    init = [(rng.standard_normal(s) * 0.02).astype(np.float32) for s in shapes]
    grads = [[(rng.standard_normal(s) * 10.0 ** rng.uniform(-4, -2)).astype(np.float32) for s in shapes]
             for _ in range(steps)]
    out = []
    for use_noalloc in (False, True):
        params = [torch.nn.Parameter(torch.from_numpy(v).to(DEV, torch.bfloat16)) for v in init]
        opt = Adakaon(params, lr=1e-3, betas=(0.9, 0.999), weight_decay=0.01, momentum_dtype=momentum_dtype,
                      momentum_4bit_block=64, **kw)
        opt.sr_seed = seed
        for k in range(steps):
            for p, g in zip(params, grads[k]):
                p.grad = torch.from_numpy(g).to(DEV, torch.bfloat16)
            if use_noalloc:
                _step_noalloc(opt)
            else:
                opt.step()
        torch.cuda.synchronize()
        out.append((params, opt))
    (pa, oa), (pb, ob) = out
    for i, (a, b) in enumerate(zip(pa, pb)):
        assert np.array_equal(_bits(a), _bits(b)), f"param {i} {tuple(a.shape)} differs"
        for key, va in oa.state[a].items():
            vb = ob.state[b][key]
            if torch.is_tensor(va):
                assert np.array_equal(_bits(va), _bits(vb)), f"param {i} state {key} differs"
            else:
                assert va == vb
    return oa


def test_noalloc_matches_step_two_calls_second_smaller():
    from kaon_amd import _lib as L

    print("[gpu] noalloc: first call, SDXL-like shapes, int8", flush=True)
    big = [[1280, 1280], [640, 320, 3, 3], [5120, 640], [1280], [77, 33], [13, 2880]]
    opt = _run(big, "int8", seed=1)
    ws_big = max(pl.info.ws_words for _k, (_ptrs, pl) in opt._plans.items())
    print("[gpu] noalloc: second call, smaller shapes, 4-bit", flush=True)
    small = [[24, 40], [8, 4, 3, 3], [33]]
    opt = _run(small, "4bit", seed=2)
    ws_small = max(pl.info.ws_words for _k, (_ptrs, pl) in opt._plans.items())
    assert ws_small < ws_big
    assert L.lib().kaon_abi_version() == L.ABI_VERSION


def test_noalloc_torch_order_matches_the_split_step():
    """reduction_order="torch" on a plan with a long clip chain (KaonLaunch.n_long > 0):
    kaon_adakaon_step runs that chain on its side stream, the allocation-free entry point
    keeps the whole step on the caller's stream; the results agree bit for bit."""
    print("[gpu] noalloc: torch order, a 14.7M-element conv beside short tensors", flush=True)
    opt = _run([[1280, 1280, 3, 3], [1280, 1280], [1280]], "int8", seed=3, reduction_order="torch")
    assert max(pl.launch.n_long for _k, (_ptrs, pl) in opt._plans.items()) == 1


def test_noalloc_rejects_a_plan_beyond_the_static_workspace():
    """The size checked is the launch's own: a real plan whose workspace exceeds the
    static array is refused before any launch, and so is a launch with no size."""
    import test_lib_cpu as C

    C.check_noalloc_refuses_oversized_plans()
