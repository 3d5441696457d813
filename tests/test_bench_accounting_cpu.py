"""CPU checks of bench.py's accounting: the shape set, the Newton-Schulz FLOP
count, the per-phase algorithmic bytes, the centralized-gradient write count and
the source-hash gate on the committed PMC traffic lines.

These figures are the numerators of every roofline the bench line reports, so
each is checked against a count made another way (an instrumented matmul, the
shape table summed by kind, the routing rule applied to meta tensors), not
against its own formula.
"""
from __future__ import annotations

import os
import shutil

import numpy as np
import pytest
import torch

import bench
from kaon_amd import workloads as W


def _meta_params(shapes, dtype=torch.bfloat16):
    out = []
    for s in shapes:
        p = torch.nn.Parameter(torch.empty(s, device="meta", dtype=dtype))
        p.grad = torch.empty(s, device="meta", dtype=dtype)
        out.append(p)
    return out


def test_sdxl_shape_set_totals():
    s = W.sdxl_shapes()
    assert len(s) == 1678
    assert len(set(s)) == 18
    assert W.n_params(s) == 2_664_150_400
    # by kind: convs, linears and vectors add up to the whole
    conv = sum(int(np.prod(x)) for x in s if len(x) == 4)
    lin = sum(int(np.prod(x)) for x in s if len(x) == 2)
    vec = sum(int(np.prod(x)) for x in s if len(x) == 1)
    assert conv == 414_720_000 and vec == 1_545_600 and conv + lin + vec == W.n_params(s)
    # the share in tensors above 2M elements (the ones the reference's foreach path steps one by one)
    big = sum(int(np.prod(x)) for x in s if np.prod(x) > 1 << 21)
    assert round(100.0 * big / W.n_params(s), 1) == 74.5


class _Counting:
    """Matmul that adds 2*M*K*N to a running FLOP total."""

    def __init__(self):
        self.flops = 0

    def mm(self, a, b):
        self.flops += 2 * a.shape[0] * a.shape[1] * b.shape[1]
        return a @ b


def _ns_counted(shape, steps):
    """One Newton-Schulz quintic run, X <- aX + (bA + cA^2) X with A = X X^T on the
    short side, through a counting matmul."""
    r = shape[0]
    c = int(np.prod(shape[1:]))
    x = np.random.default_rng(0).standard_normal((r, c))
    if r > c:
        x = x.T
    x = x / np.linalg.norm(x)
    cnt = _Counting()
    for _ in range(steps):
        a = cnt.mm(x, x.T)
        b = -4.7750 * a + 2.0315 * cnt.mm(a, a)
        x = 3.4445 * x + cnt.mm(b, x)
    return cnt.flops


@pytest.mark.parametrize("shape", [(6, 10), (10, 6), (4, 3, 3, 3), (12, 2, 3, 3), (7, 7)])
@pytest.mark.parametrize("steps", [1, 2, 5])
def test_ns_flops_matches_an_instrumented_run(shape, steps):
    assert bench.ns_flops([shape], steps) == _ns_counted(shape, steps)


def test_ns_flops_skips_vectors_and_sums_over_the_set():
    assert bench.ns_flops([(1280,), (5120,)], 2) == 0.0
    shapes = [(6, 10), (5,), (4, 3, 3, 3)]
    assert bench.ns_flops(shapes, 3) == _ns_counted((6, 10), 3) + _ns_counted((4, 3, 3, 3), 3)
    # the figure the adamuon_int8 roofline is priced on
    assert round(bench.ns_flops(W.sdxl_shapes(), 2) / 1e12, 1) == 32.2


def test_phase_bytes_per_param():
    # apply: g read (2), p read + write (4), momentum read + write (2 b_m)
    assert bench.phase_bytes(6, 1.0, False) == 8.0
    assert bench.phase_bytes(6, 0.5, False) == 7.0
    assert bench.phase_bytes(6, 2.0, False) == 10.0
    # keep count: g and m read, p read too when weight decay enters the mask
    assert bench.phase_bytes(5, 1.0, False) == 3.0
    assert bench.phase_bytes(5, 1.0, True) == 5.0
    # row statistics and clip sums read g once; the finalize and divisor phases touch no per-param data
    assert bench.phase_bytes(1, 1.0, False) == bench.phase_bytes(3, 1.0, False) == 2.0
    assert bench.phase_bytes(2, 1.0, False) == bench.phase_bytes(4, 1.0, False) == 0.0
    # AdaPNM reads its negative momentum in the clip-sum, keep-count and apply passes
    assert bench.phase_bytes(6, 1.0, False, "adapnm") == 9.0
    # MSAM's norm (m read) and climb (m read, p read + write) passes
    assert bench.phase_bytes(13, 1.0, False, "msam") == 1.0
    assert bench.phase_bytes(14, 1.0, False, "msam") == 5.0
    # KProdigy, memory-lean: sliced statistics over slice_p = 11
    w = bench.WORKLOADS["kprodigy_int8_factored"]
    assert bench.phase_bytes(11, 1.0, False, "kprodigy", w) == pytest.approx(4.0 + 16.0 / 11)
    assert bench.phase_bytes(12, 1.0, False, "kprodigy", w) == 7.0


def test_gc_written_elems_small_set():
    shapes = [(64, 32), (8, 4, 3, 3), (32,)]
    ps = _meta_params(shapes, torch.float32)
    two_d = 64 * 32 + 8 * 4 * 9
    # Lion stores every 2-D+ gradient back centralized
    assert bench.gc_written_elems(bench.make_opt("lion_int8", ps), "lion_int8") == two_d
    # fused Adakaon with int8 momentum: only the convs go to the native path
    assert bench.gc_written_elems(bench.make_opt("adakaon_int8", ps), "adakaon_int8") == 8 * 4 * 9
    from kaon_amd import Adakaon
    unfused = Adakaon(ps, lr=1e-4, momentum_dtype="int8", fused=False)
    assert bench.gc_written_elems(unfused, "adakaon_int8") == two_d
    off = Adakaon(ps, lr=1e-4, momentum_dtype="int8", fused=False, gradient_centralization=False)
    assert bench.gc_written_elems(off, "adakaon_int8") == 0
    # AdaMuon's headline kernels do not store the gradient
    assert bench.gc_written_elems(bench.make_opt("adamuon_int8", ps), "adamuon_int8") == 0


def test_gc_written_elems_on_the_sdxl_set():
    """The headline apply's algorithmic bytes: 8 B/param plus 2 B per centralized
    gradient element the fused step stores (the convs)."""
    s = W.sdxl_shapes()
    ps = _meta_params(s)
    conv = sum(int(np.prod(x)) for x in s if len(x) == 4)
    assert bench.gc_written_elems(bench.make_opt("adakaon_int8", ps), "adakaon_int8") == conv
    assert bench.gc_written_elems(bench.make_opt("lion_int8", ps), "lion_int8") == \
        sum(int(np.prod(x)) for x in s if len(x) >= 2)
    apply_gb = (bench.phase_bytes(6, 1.0, False) * W.n_params(s) + 2.0 * conv) / 1e9
    assert apply_gb == pytest.approx(22.14, abs=0.005)


def test_kernel_source_hash_ignores_comments(tmp_path, monkeypatch):
    for rel in bench.KERNEL_SOURCES:
        dst = tmp_path / rel
        dst.parent.mkdir(parents=True, exist_ok=True)
        shutil.copy(os.path.join(bench.ROOT, rel), dst)
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    h0 = bench.kernel_source_hash()
    f = tmp_path / bench.KERNEL_SOURCES[0]
    text = f.read_text()
    f.write_text("// a comment line\n\n/* a block\n comment */\n" + text.replace("\n", "  // trailing\n", 1))
    assert bench.kernel_source_hash() == h0
    f.write_text(text + "\nstatic int unused_probe = 1;\n")
    assert bench.kernel_source_hash() != h0


def test_measured_traffic_reads_only_the_matching_source(monkeypatch):
    import glob
    import re

    lines = []
    for path in sorted(glob.glob(os.path.join(bench.ROOT, "profiles", "*_pmc.md"))):
        with open(path) as fh:
            lines += [ln.strip() for ln in fh if ln.startswith("traffic:")]
    assert lines, "no traffic lines in the committed PMC summaries"
    pat = re.compile(r"traffic: workload=(\S+) phase=(\d+) kernel=\S+ bytes=(\S+) source=(\w+)$")
    for ln in lines:
        m = pat.match(ln)
        assert m, ln
        assert m.group(1) in bench.WORKLOADS
        monkeypatch.setattr(bench, "kernel_source_hash", lambda src=m.group(4): src)
        assert bench.measured_traffic(m.group(1), int(m.group(2))) == float(m.group(3))
        monkeypatch.setattr(bench, "kernel_source_hash", lambda: "0" * 16)
        assert bench.measured_traffic(m.group(1), int(m.group(2))) is None
