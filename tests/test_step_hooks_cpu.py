"""The optimizers' step() runs torch.optim's step hooks as torch.optim.Optimizer's
own step wrapper does (which it replaces: ``step.hooked``): global then instance
pre-hooks, which may replace the arguments, the step, then instance and global
post-hooks, each called with (optimizer, args, kwargs).  Checked against the
wrapper's behaviour on torch.optim.SGD with the same hooks.  The step body is
replaced by a recorder, so no device is needed."""
import pytest
import torch
from torch.optim.optimizer import register_optimizer_step_post_hook, register_optimizer_step_pre_hook

import kaon_amd as K

OPTS = {
    "Adakaon": lambda ps: K.Adakaon(ps, lr=1e-3),
    "Lion": lambda ps: K.Lion(ps, lr=1e-4),
    "AdaMuon": lambda ps: K.AdaMuon(ps, lr=2e-2),
    "AdaPNM": lambda ps: K.AdaPNM(ps, lr=1e-3),
    "KProdigy": lambda ps: K.KProdigy(ps, lr=1.0),
}


def _trace(opt, body):
    log = []
    hs = [register_optimizer_step_pre_hook(lambda o, a, k: log.append(("gpre", len(a), dict(k)))),
          opt.register_step_pre_hook(lambda o, a, k: log.append(("pre", len(a), dict(k)))),
          opt.register_step_post_hook(lambda o, a, k: log.append(("post", len(a), dict(k)))),
          register_optimizer_step_post_hook(lambda o, a, k: log.append(("gpost", len(a), dict(k))))]
    try:
        out = body(log)
    finally:
        for h in hs:
            h.remove()
    return log, out


@pytest.mark.parametrize("name", sorted(OPTS))
def test_step_hooks_match_torch_wrapper(name):
    ps = [torch.nn.Parameter(torch.zeros(4, 4))]
    ref = torch.optim.SGD([torch.nn.Parameter(torch.zeros(4, 4))], lr=0.1)
    opt = OPTS[name](ps)
    assert getattr(type(opt).step, "hooked", False)

    def run(o, log):
        calls = []
        if o is opt:
            o._step_impl = lambda *a, **k: (calls.append((a, k)), log.append(("step",)), 7)[2]
        out1 = o.step()
        out2 = o.step(lambda: 3.0)
        return calls, out1, out2

    log_ref, _ = _trace(ref, lambda log: ref.step())
    log_ref2, _ = _trace(ref, lambda log: ref.step(lambda: 3.0))
    log, (calls, out1, out2) = _trace(opt, lambda log: run(opt, log))
    no_step = [e for e in log if e[0] != "step"]
    assert no_step == log_ref + log_ref2
    assert [e[0] for e in log] == ["gpre", "pre", "step", "post", "gpost"] * 2
    assert out1 == 7 and out2 == 7
    assert calls[0] == ((), {}) and len(calls[1][0]) == 1 and calls[1][0][0]() == 3.0


def test_pre_hook_replaces_the_arguments():
    opt = K.Adakaon([torch.nn.Parameter(torch.zeros(4, 4))], lr=1e-3)
    seen = []
    opt._step_impl = lambda *a, **k: seen.append((a, k))
    h = opt.register_step_pre_hook(lambda o, a, k: (a, {"closure": None}))
    opt.step()
    h.remove()
    h = opt.register_step_pre_hook(lambda o, a, k: "bad")
    with pytest.raises(RuntimeError, match="must return None or a tuple"):
        opt.step()
    h.remove()
    assert seen == [((), {"closure": None})]
