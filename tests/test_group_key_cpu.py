"""The launch-cache key of a parameter group (kaon_amd._keys, native helper
_kaon_key): which params a step takes, and a key that changes whenever a cached
plan would no longer describe them.  CPU tensors: the helper reads only host
metadata (storage pointers, dtype, layout)."""
import torch

from kaon_amd import _keys as K


def _params(n=12, shape=(8, 16)):
    ps = [torch.nn.Parameter(torch.zeros(shape)) for _ in range(n)]
    for i, p in enumerate(ps):
        if i % 5 != 3:
            p.grad = torch.randn(shape)
    return ps


def test_kept_params_are_those_with_a_grad_in_order():
    ps = _params()
    kept, key = K.group_key(ps)
    assert kept == [p for p in ps if p.grad is not None]
    assert all(a is b for a, b in zip(kept, [p for p in ps if p.grad is not None]))
    assert len(key) == 19 * len(kept)
    assert K.group_key([]) == ([], b"")


def test_key_is_stable_while_nothing_changes():
    ps = _params()
    _, k0 = K.group_key(ps)
    for p in ps:
        if p.grad is not None:
            p.grad.mul_(2.0)  # values change, storage does not
    assert K.group_key(ps)[1] == k0


def test_key_changes_with_everything_a_plan_depends_on():
    ps = _params()
    base = K.group_key(ps)[1]
    i = 0

    def changed(mutate):
        q = _params()
        for a, b in zip(q, ps):
            a.data = b.data
            a.grad = b.grad
        mutate(q)
        return K.group_key(q)[1] != base

    assert changed(lambda q: setattr(q[i], "grad", q[i].grad.clone()))                  # new grad storage
    assert changed(lambda q: (setattr(q[i], "grad_dtype", None),                         # grad dtype
                              setattr(q[i], "grad", q[i].grad.to(torch.bfloat16))))
    assert changed(lambda q: setattr(q[i], "grad", torch.randn(16, 8).t()))             # grad not contiguous
    assert changed(lambda q: setattr(q[i], "data", q[i].data.clone()))                  # param storage
    assert changed(lambda q: setattr(q[3], "grad", torch.randn(8, 16)))                 # a param gains a grad
    assert changed(lambda q: setattr(q[i], "grad", None))                               # a param loses it
    sp = torch.randn(8, 16).to_sparse()
    assert changed(lambda q: setattr(q[i], "grad", sp))                                 # a sparse grad


def test_non_tensors_are_refused():
    try:
        K.group_key([object()])
    except TypeError:
        return
    raise AssertionError("expected a TypeError")


def test_any_sequence_or_iterable_and_gradless_runs():
    """Tuples and generators give the same result as lists; params without a grad at the
    start, middle and end are left out, and the key's records stay aligned."""
    ps = _params(20)
    ps[0].grad = None
    ps[19].grad = None
    want = [p for p in ps if p.grad is not None]
    for arg in (ps, tuple(ps), (p for p in ps)):
        kept, key = K.group_key(arg)
        assert type(kept) is list and all(a is b for a, b in zip(kept, want)) and len(kept) == len(want)
        assert key == K.group_key(want)[1]
    # every record: param pointer, grad pointer, then dtype / contiguity / sparsity tags
    kept, key = K.group_key(ps)
    for j, p in enumerate(kept):
        rec = key[19 * j:19 * (j + 1)]
        assert int.from_bytes(rec[0:8], "little") == p.data_ptr()
        assert int.from_bytes(rec[8:16], "little") == p.grad.data_ptr()
        assert rec[17] == 1 and rec[18] == 0
    none = [torch.nn.Parameter(torch.zeros(2)) for _ in range(3)]
    assert K.group_key(none) == ([], b"")


def test_a_refused_element_after_kept_params_leaves_them_intact():
    ps = _params(4)
    refs = [p for p in ps]
    for bad in ([ps[0], ps[1], 3], (ps[2], "x")):
        try:
            K.group_key(bad)
        except TypeError:
            pass
        else:
            raise AssertionError("expected a TypeError")
    assert all(a is b for a, b in zip(ps, refs))
    assert K.group_key(ps)[0] == [p for p in ps if p.grad is not None]


def test_no_reference_leak():
    import sys

    ps = _params(8)
    before = [sys.getrefcount(p) for p in ps]
    for _ in range(200):
        K.group_key(ps)
        try:
            K.group_key(ps + [None])
        except TypeError:
            pass
    assert [sys.getrefcount(p) for p in ps] == before
