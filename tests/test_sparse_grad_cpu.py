"""A sparse gradient is refused with RuntimeError before any device work, by every
optimizer (the reference's behaviour: tests/test_lion.py:333-338 there), and the
optimizer state is left untouched."""
import pytest
import torch

import kaon_amd as K

OPTS = {
    "Adakaon": lambda ps: K.Adakaon(ps, lr=1e-3),
    "Lion": lambda ps: K.Lion(ps, lr=1e-4),
    "Nekaon": lambda ps: K.Nekaon(ps, lr=1e-4),
    "AdaMuon": lambda ps: K.AdaMuon(ps, lr=2e-2),
    "AdaPNM": lambda ps: K.AdaPNM(ps, lr=1e-3),
    "KProdigy": lambda ps: K.KProdigy(ps, lr=1.0),
    "MSAM": lambda ps: K.MSAM(ps, lr=1e-3),
}


@pytest.mark.parametrize("name", sorted(OPTS))
def test_sparse_grad_is_refused(name):
    p = torch.nn.Parameter(torch.zeros(8, 16))
    q = torch.nn.Parameter(torch.zeros(8, 16))
    opt = OPTS[name]([p, q])
    q.grad = torch.zeros(8, 16)
    p.grad = torch.zeros(8, 16).to_sparse()
    with pytest.raises(RuntimeError, match="sparse"):
        opt.step()
    inner = getattr(opt, "inner", opt)
    assert all(len(inner.state[t]) == 0 for t in (p, q))
