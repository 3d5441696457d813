"""Optimizer-step throughput on a synthetic SDXL-UNet-shaped 2.664B-param bf16 set, 1 GPU.

Metric: Gparam/s and % of the HBM roofline per optimizer step.
Default workload = BASELINE configs[2]: Adakaon, betas (0.9, 0.999), int8
momentum, cautious, gradient centralization, stochastic-rounding bf16 writes,
lr 1e-4 (the configuration the metric is quoted on).  ``--workload lion_int8``
(configs[1]), ``nekaon_4bit_b64`` / ``nekaon_4bit_b256`` (configs[3]'s two block
sizes; ``nekaon_4bit`` keeps Nekaon's default 128), ``adamuon_int8``
(configs[4]) and the adjacent optimizers (``adapnm_*``, ``kprodigy_*``,
``msam_int8``, ``lora_bag``) select the others.

A "step" is one ``optimizer.step()`` over all 1,678 tensors with the params,
grads and optimizer state resident in HBM.  W untimed warmup steps (the first
one builds the plan and the state), then K steps between two
``torch.cuda.synchronize()`` calls.

Besides the JSON line's ``value`` (Gparam/s) the line carries
* ``roofline``: the dominant kernel of the step (largest share of the step
  time), its algorithmic HBM bytes per launch (bytes/param of that kernel x
  params) divided by its average duration, measured with HIP events on the
  launch stream (one phase at a time through ``kaon_adakaon_phases``);
  ``traffic`` is the HBM bytes per launch that rocprofv3's FETCH_SIZE and
  WRITE_SIZE counters measured for that kernel, read from the committed
  profiles/*_pmc.md summary only when the summary's source hash matches the
  current kernel sources (null otherwise);
* ``step_roofline``: the whole step at the algorithmic 2 + 4 + 2*b_m bytes/param
  (g read, p read+write, momentum read+write), against 8 TB/s, against a copy
  kernel measured on the same device (1:1 read:write) and against a kernel
  with the apply's own access mix (``kaon_apply_ceiling``: bf16 g and p and
  int8 m read, p and m written, 5:3);
* ``lora_bag`` (default workload): ms per step of the launch-bound regime, the
  reference's LoRA proxy bag of 512 fp32 [8, 16] tensors;
* ``torch_order`` (Adakaon / Lion workloads): the same step with
  ``reduction_order="torch"``, whose fp32 sums follow torch CPU's order and so
  give the reference's bits; ms per step and its phases;
* ``cpu_baseline``: the reference's CPU path, its native foreach step restated
  in torch (oracle/torch_foreach.py, pinned bit for bit against the reference's
  fixtures), on the job's host cores over a fixed sample of the set (every 2nd
  tensor by default, ``--cpu-stride 1`` for the whole set), the median of three
  steps after a warmup; ``cpu_oracle_baseline`` beside it is the C oracle
  (oracle/kaon_oracle.c) on the same host (at most 16 threads).  4-bit
  workloads and the other optimizers report the C oracle as ``cpu_baseline``.
  A reported baseline, not the target.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "k-optimizers_amd"))

METRIC = "Gparam/s + % HBM roofline per optimizer step, 2.6B bf16 params, 1 GPU"
HBM_PEAK_GBS = 8000.0

WORKLOADS = {
    "adakaon_int8": dict(desc="configs[2]: Adakaon betas=(0.9,0.999) int8 momentum, cautious, GC, SR bf16, lr 1e-4, "
                              "fused=True",
                         opt="adakaon", kw=dict(lr=1e-4, betas=(0.9, 0.999), momentum_dtype="int8", fused=True),
                         bm=1.0),
    "lion_int8": dict(desc="configs[1]: Lion betas=(0.95,0.98) int8 momentum, cautious, GC, SR bf16, lr 2e-4, "
                           "p.grad left centralized as the reference's Lion leaves it",
                      opt="lion", kw=dict(lr=2e-4, betas=(0.95, 0.98), momentum_dtype="int8"), bm=1.0),
    "nekaon_4bit": dict(desc="configs[3]: Nekaon k=1.5 beta1=0.2 4-bit block 128, wd 0.1, cautious, GC, SR bf16, "
                             "lr 1e-4, 1% Student-t outliers, fused=True", opt="nekaon",
                        kw=dict(lr=1e-4, betas=(0.2, 0.999), momentum_dtype="4bit", momentum_4bit_block=128,
                                fused=True),
                        bm=0.5, outliers=0.01),
    # configs[3] names block sizes 64 and 256 (the default workload above keeps Nekaon's default 128)
    "nekaon_4bit_b64": dict(desc="configs[3]: Nekaon k=1.5 beta1=0.2 4-bit block 64, wd 0.1, cautious, GC, SR bf16, "
                                 "lr 1e-4, 1% Student-t outliers, fused=True", opt="nekaon",
                            kw=dict(lr=1e-4, betas=(0.2, 0.999), momentum_dtype="4bit", momentum_4bit_block=64,
                                    fused=True),
                            bm=0.5, outliers=0.01),
    "nekaon_4bit_b256": dict(desc="configs[3]: Nekaon k=1.5 beta1=0.2 4-bit block 256, wd 0.1, cautious, GC, SR "
                                  "bf16, lr 1e-4, 1% Student-t outliers, fused=True", opt="nekaon",
                             kw=dict(lr=1e-4, betas=(0.2, 0.999), momentum_dtype="4bit", momentum_4bit_block=256,
                                     fused=True),
                             bm=0.5, outliers=0.01),
    "adamuon_int8": dict(desc="configs[4]: AdaMuon ns_steps=2, betas=(0.95,0.999), int8 momentum, factored 2nd "
                              "moment, cautious, SR bf16, lr 2e-2; Newton-Schulz on every 2-D / conv matrix, 1-D "
                              "params on the Adakaon path", opt="adamuon",
                         kw=dict(lr=2e-2, betas=(0.95, 0.999), momentum_dtype="int8", ns_steps=2), bm=1.0),
    # AdaPNM (src/kaon/adapnm.py): two momenta, the positive one read and
    # written, the negative one read (b_neg), on the same SDXL set
    "adapnm_int8": dict(desc="AdaPNM betas=(0.8,0.999) beta0=0.5, two int8 momenta, factored 2nd moment, cautious, "
                             "GC, SR bf16, lr 1e-4, fused=True", opt="adapnm",
                        kw=dict(lr=1e-4, betas=(0.8, 0.999), beta0=0.5, momentum_dtype="int8", fused=True), bm=1.0,
                        b_neg=1.0),
    "adapnm_bf16": dict(desc="AdaPNM defaults: betas=(0.8,0.999) beta0=0.5, two bf16 momenta, factored 2nd moment, "
                             "cautious, GC, SR bf16, lr 1e-4, fused=True", opt="adapnm",
                        kw=dict(lr=1e-4, betas=(0.8, 0.999), beta0=0.5, momentum_dtype="bfloat16", fused=True), bm=2.0,
                        b_neg=2.0),
    # KProdigy (src/kaon/kprodigy.py): two passes around a cross-tensor D
    # estimate; b_extra = the fp32 v (read + write) and the sliced s (read + write) and p0 (read)
    "kprodigy_bf16": dict(desc="KProdigy defaults: lr 1.0, d0 1e-6, betas=(0.9,0.999), bf16 momentum, full fp32 "
                               "second moment, slice_p 1, GC, SR bf16", opt="kprodigy",
                          kw=dict(lr=1.0, betas=(0.9, 0.999), momentum_dtype="bfloat16"), bm=2.0,
                          b_extra=8.0 + 12.0, pd_slice=1, pd_full_v=True),
    "kprodigy_int8_factored": dict(desc="KProdigy memory-lean: lr 1.0, int8 momentum, factored second moment, "
                                        "slice_p 11, GC, SR bf16", opt="kprodigy",
                                   kw=dict(lr=1.0, betas=(0.9, 0.999), momentum_dtype="int8",
                                           second_moment="factored", slice_p=11), bm=1.0,
                                   b_extra=12.0 / 11.0, pd_slice=11, pd_full_v=False),
    # MSAM norm="global" over Adakaon (src/kaon/msam.py): the removal rides in
    # Adakaon's apply; b_extra = the norm pass (m read) and the climb pass (m read, p read + write)
    "msam_int8": dict(desc="MSAM rho=0.3 norm='global' over Adakaon betas=(0.9,0.999) int8 momentum, cautious, GC, "
                           "SR bf16, lr 1e-4, fused=True", opt="msam",
                      kw=dict(lr=1e-4, rho=0.3, betas=(0.9, 0.999), momentum_dtype="int8", fused=True), bm=1.0,
                      b_extra=1.0 + 4.0 + 1.0),
    # the launch-bound regime: the reference's LoRA proxy bag (benchmarks/proxy/harness.py:117-127:
    # 512 tensors [8, 16], fp32) stepped by Adakaon with bf16 momentum, the configuration its
    # control ranking lists as "Adakaon-bf16-fused" (benchmarks/control/RANKINGS.md:83)
    "lora_bag": dict(desc="LoRA bag: 512 x [8,16] fp32 params and grads, Adakaon bf16 momentum, cautious, GC, "
                          "lr 1e-4, fused=True", opt="adakaon",
                     kw=dict(lr=1e-4, betas=(0.9, 0.999), momentum_dtype="bfloat16", fused=True),
                     bm=2.0, shapes=[(8, 16)] * 512, pdtype="f32"),
}
LORA_METRIC = "ms per optimizer step, LoRA bag 512 x [8,16] fp32, 1 GPU"
BF16_MFMA_PEAK_TFLOPS = 2500.0

# algorithmic HBM bytes per param of each phase kernel (bf16 g/p, b_m momentum bytes)
PHASE_NAMES = {1: "row_stats", 2: "finalize", 3: "clip_sums", 4: "clip_divisor", 5: "keep_count", 6: "apply",
               8: "momentum", 9: "newton_schulz", 11: "pass1_moments_and_d_stats", 12: "pass2_update",
               13: "momentum_sumsq", 14: "climb"}


def phase_bytes(phase: int, bm: float, wd: bool, opt: str = "adakaon", w: dict | None = None) -> float:
    if opt == "kprodigy":
        # pass 1: g, m (read + write), v (read + write); then the sliced g, p, fp32 p0 and the
        # fp32 s (read + write) for the D statistics; pass 2: g, m, v, p (read + write)
        full = 1.0 if w and w.get("pd_full_v") else 0.0
        sl = (w or {}).get("pd_slice", 1)
        return {11: 2.0 + 2.0 * bm + 8.0 * full + 16.0 / sl, 12: 2.0 + bm + 4.0 * full + 4.0}.get(phase, 0.0)
    if opt == "msam":
        # the Adakaon phases (the removal reads the momentum the update reads anyway), then
        # the norm (m read) and the climb (m read, p read + write)
        if phase in (13, 14):
            return {13: bm, 14: 4.0 + bm}[phase]
    if opt == "adapnm":
        # both momenta are read by the clip-sum, keep-count and apply passes
        return {1: 2.0, 3: 2.0 + 2.0 * bm, 5: 2.0 + 2.0 * bm, 6: 6.0 + 3.0 * bm}.get(phase, 0.0)
    if phase in (1, 3):
        return 2.0
    if phase == 5:
        return 2.0 + bm + (2.0 if wd else 0.0)
    if phase == 6:
        return 2.0 + 4.0 + 2.0 * bm
    return 0.0


KERNEL_SOURCES = ("k-optimizers_amd/csrc/kaon_step.hip", "k-optimizers_amd/csrc/kaon_fast.hip",
                  "k-optimizers_amd/csrc/kaon_common.h", "k-optimizers_amd/csrc/kaon_device.h",
                  "k-optimizers_amd/csrc/kaon_ns.hip", "k-optimizers_amd/csrc/kaon_plan.cpp")


def kernel_source_hash() -> str:
    """sha256 (first 16 hex digits) of the step kernels' source files with their
    comments and blank lines removed, the key a committed PMC summary records for
    the build it measured (an edit to a comment does not invalidate it)."""
    import hashlib
    import re

    h = hashlib.sha256()
    for rel in KERNEL_SOURCES:
        with open(os.path.join(ROOT, rel), encoding="utf-8") as fh:
            text = fh.read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        lines = [ln.rstrip() for ln in text.splitlines() if ln.strip()]
        h.update("\n".join(lines).encode())
    return h.hexdigest()[:16]


def measured_traffic(workload: str, phase: int) -> float | None:
    """HBM bytes per launch of a phase kernel, from the rocprofv3 PMC summaries
    committed under profiles/ (FETCH_SIZE and WRITE_SIZE, each scaled by what
    the counter reads for a copy kernel of known size).  Only a summary taken
    with the current kernel sources counts (its ``source=`` hash must equal
    kernel_source_hash()); otherwise None."""
    import glob
    import re

    src = kernel_source_hash()
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*_pmc.md"))):
        with open(path) as fh:
            for line in fh:
                m = re.match(r"traffic: workload=(\S+) phase=(\d+) kernel=\S+ bytes=(\S+) source=(\w+)", line.strip())
                if m and m.group(1) == workload and int(m.group(2)) == phase and m.group(4) == src:
                    return float(m.group(3))
    return None


def make_opt(name, params):
    from kaon_amd import MSAM, AdaMuon, AdaPNM, Adakaon, KProdigy, Lion, Nekaon

    w = WORKLOADS[name]
    if w["opt"] == "msam":
        return MSAM(params, **w["kw"])
    if w["opt"] == "adapnm":
        return AdaPNM(params, **w["kw"])
    if w["opt"] == "kprodigy":
        return KProdigy(params, **w["kw"])
    if w["opt"] == "adakaon":
        return Adakaon(params, **w["kw"])
    if w["opt"] == "lion":
        return Lion(params, **w["kw"])
    if w["opt"] == "adamuon":
        return AdaMuon(params, **w["kw"])
    return Nekaon(params, **w["kw"])


def gc_written_elems(opt, name) -> int:
    """Elements whose p.grad the step's apply stores back centralized (2-D+ params only).

    Lion writes every 2-D+ gradient back; Adakaon (and the Nekaon / MSAM steps over
    it) does so on its native path and, under ``fused=True``, only for the params
    the reference's fused step routes to its native path (``fused_routes_native``).
    Other optimizers' headline kernels do not store the gradient."""
    from kaon_amd.adakaon import fused_routes_native

    w = WORKLOADS[name]
    inner = getattr(opt, "inner", opt)  # Nekaon / MSAM step an inner Adakaon
    if w["opt"] not in ("lion", "adakaon", "nekaon", "msam") or \
            not getattr(inner, "centralize_grads_in_place", False):
        return 0
    fused = w["opt"] != "lion" and getattr(inner, "_fused", False)
    n = 0
    for g in opt.param_groups:
        if not g.get("gradient_centralization", True):
            continue
        for p in g["params"]:
            if p.ndim < 2:
                continue
            if fused and not fused_routes_native(p, g, inner._fused_tile_cap):
                continue
            n += p.numel()
    return n


def ns_flops(shapes, steps: int) -> float:
    """Newton-Schulz FLOPs per optimizer step: sum over 2-D / conv matrices of
    steps * (4 m^2 n + 2 m^3), m = min(R, C), n = max(R, C) (x x^T, A A, B x)."""
    tot = 0.0
    for s in shapes:
        if len(s) < 2:
            continue
        r = s[0]
        c = 1
        for d in s[1:]:
            c *= d
        m, n = min(r, c), max(r, c)
        tot += steps * (4.0 * m * m * n + 2.0 * m ** 3)
    return tot


def ns_library_ms(dev, shapes, steps: int, reps: int = 5) -> dict:
    """The same Newton-Schulz products through the vendor GEMM (torch.bmm: hipBLASLt /
    rocBLAS), batched per distinct (m, n): X X^T ([b,m,n] x [b,n,m]), A A ([b,m,m] x
    [b,m,m]) and B X ([b,m,m] x [b,m,n]), operands contiguous, no epilogues.  Their
    summed time per step is a library composition of the phase to set beside the
    HIP kernels (which also exploit the symmetry of X X^T and A A, and fuse the
    b A + c A A and a X + B X epilogues).  Random bf16 operands: GEMM time does not
    depend on the values."""
    import torch

    groups: dict[tuple[int, int], int] = {}
    for s in shapes:
        if len(s) < 2:
            continue
        c = 1
        for d in s[1:]:
            c *= d
        m, n = min(s[0], c), max(s[0], c)
        groups[(m, n)] = groups.get((m, n), 0) + 1
    per = {"xxt": 0.0, "aa": 0.0, "bx": 0.0}
    flops = 0.0
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for (m, n), b in sorted(groups.items()):
        for name, (k, cols, rows) in (("xxt", (n, m, m)), ("aa", (m, m, m)), ("bx", (m, n, m))):
            a = torch.randn(b, rows, k, device=dev, dtype=torch.bfloat16)
            x = torch.randn(b, k, cols, device=dev, dtype=torch.bfloat16)
            o = torch.empty(b, rows, cols, device=dev, dtype=torch.bfloat16)
            torch.bmm(a, x, out=o)
            torch.cuda.synchronize()
            e0.record()
            for _ in range(reps):
                torch.bmm(a, x, out=o)
            e1.record()
            torch.cuda.synchronize()
            per[name] += e0.elapsed_time(e1) / reps
            flops += 2.0 * b * rows * k * cols
            del a, x, o
    torch.cuda.empty_cache()
    tot = steps * sum(per.values())
    return {"ms_per_step": round(tot, 3), "tflops": round(steps * flops / (tot * 1e-3) / 1e12, 1),
            "ms_per_iteration": {k: round(v, 3) for k, v in per.items()},
            "note": "torch.bmm per distinct (m, n) of the set, products only (no symmetry, no epilogues)"}


def copy_ceiling_gbs(dev, nbytes=4 << 30, reps=10) -> float:
    import torch
    from kaon_amd import _lib

    src = torch.empty(nbytes // 2, dtype=torch.int16, device=dev)
    src.fill_(1)
    dst = torch.empty_like(src)
    s = torch.cuda.current_stream(dev).cuda_stream
    lib = _lib.lib()
    _lib.check(lib.kaon_copy(src.data_ptr(), dst.data_ptr(), nbytes, s), "kaon_copy")
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(reps):
        lib.kaon_copy(src.data_ptr(), dst.data_ptr(), nbytes, s)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / reps
    del src, dst
    return 2.0 * nbytes / (ms * 1e-3) / 1e9


def apply_mix_ceiling_gbs(dev, n=512 << 20, reps=10) -> float:
    """kaon_apply_ceiling: the apply's streams (bf16 g and p read, int8 m read,
    p and m written; 8 B per element) without its arithmetic, n elements."""
    import torch
    from kaon_amd import _lib

    g = torch.ones(n, dtype=torch.int16, device=dev)
    p = torch.ones(n, dtype=torch.int16, device=dev)
    m = torch.zeros(n, dtype=torch.int8, device=dev)
    s = torch.cuda.current_stream(dev).cuda_stream
    lib = _lib.lib()
    _lib.check(lib.kaon_apply_ceiling(g.data_ptr(), p.data_ptr(), m.data_ptr(), n, s), "kaon_apply_ceiling")
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(reps):
        lib.kaon_apply_ceiling(g.data_ptr(), p.data_ptr(), m.data_ptr(), n, s)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / reps
    del g, p, m
    return 8.0 * n / (ms * 1e-3) / 1e9


def lora_bag_ms(dev, steps=200, warmup=5) -> float:
    """ms per step of the launch-bound regime: the reference's LoRA proxy bag
    (512 fp32 [8, 16] tensors, Adakaon with bf16 momentum), HIP events over 200
    steps (about 8 ms: fewer would let one pause of the host thread weigh on the
    mean of a host-bound step)."""
    import torch
    from kaon_amd import workloads

    w = WORKLOADS["lora_bag"]
    params = workloads.make_params(w["shapes"], dev, seed=0, dtype=torch.float32)
    opt = make_opt("lora_bag", params)
    for _ in range(warmup):
        opt.step()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        opt.step()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps


def phase_breakdown(opt, name, reps=5) -> dict[int, float]:
    """Average duration (ms) of each phase kernel, HIP events on the launch stream."""
    import torch
    from kaon_amd import _lib

    inner = getattr(opt, "inner", opt)
    lib = _lib.lib()
    out: dict[int, list[float]] = {}  # per phase: [sum over plans] per rep
    for key, (_ptrs, plan) in inner._plans.items():
        gid, pdt, gdt = key[:3]
        group = inner.param_groups[gid]
        if WORKLOADS[name]["opt"] == "kprodigy":
            # the two passes with the group's current d (the host D update between them is a
            # fold of two floats per tensor)
            import math as _m
            d = group["d"]
            c = {"d": d, "dlr": d * group["lr"], "beta3": _m.sqrt(group["betas"][1]), "should_update_d": True,
                 "alpha_s": d * group["lr"] * d / group["d0"], "d_new": d}
            hp = inner._hyper(group, pdt, gdt, c)
            s = torch.cuda.current_stream().cuda_stream
            for r in range(reps):
                for ph, fn in ((11, lib.kaon_kprodigy_pass1), (12, lib.kaon_kprodigy_pass2)):
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                    _lib.check(fn(ctypes.byref(plan.launch), ctypes.byref(hp), s), "pass")
                    e1.record()
                    torch.cuda.synchronize()
                    acc = out.setdefault(ph, [0.0] * reps)
                    acc[r] += e0.elapsed_time(e1)
            continue
        if WORKLOADS[name]["opt"] == "adamuon":
            if key[3] != 2:
                continue  # the 1-D params' Adakaon plan: a few microseconds
            hp = inner._hyper(group, pdt, gdt)
            fn, phases = lib.kaon_adamuon_phases, (8, 9, 1, 2, 3, 4, 5, 6)
        elif WORKLOADS[name]["opt"] == "lion":
            hp = inner._hyper(group, pdt, gdt)
            fn, phases = lib.kaon_lion_phases, (1, 5, 6)
        elif WORKLOADS[name]["opt"] == "adapnm":
            hp = inner._hyper(group, pdt, gdt)
            fn, phases = lib.kaon_adapnm_phases, (1, 2, 3, 4, 5, 6)
        else:
            nk = None
            if WORKLOADS[name]["opt"] == "nekaon":
                nk = {"remove": True, "bound_old": dict(opt._eclamp), "k": opt.k, "eclamp": {}}
            if WORKLOADS[name]["opt"] == "msam":
                nk = {"remove": True, "bound_old": {gid: float("inf")}, "k": -opt.rho / (opt._mnorm + opt.eps),
                      "climb": False, "eclamp": {}}
            hp = inner._hyper(group, pdt, gdt, nk, gid)
            fn, phases = lib.kaon_adakaon_phases, (1, 2, 3, 4, 5, 6)
        s = torch.cuda.current_stream().cuda_stream
        for r in range(reps):
            for ph in phases:
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                _lib.check(fn(ctypes.byref(plan.launch), ctypes.byref(hp), 1 << ph, s), "phase")
                e1.record()
                torch.cuda.synchronize()
                acc = out.setdefault(ph, [0.0] * reps)
                acc[r] += e0.elapsed_time(e1)
    if WORKLOADS[name]["opt"] == "msam":
        # the norm and the climb passes over the momentum plans
        s = torch.cuda.current_stream().cuda_stream
        for gid, pdt, plan, _tids, _idx in opt._momentum_plans():
            h = opt._hyper(gid, pdt)
            f = opt.rho / (opt._mnorm + opt.eps)
            for r in range(reps):
                for ph in (13, 14):
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                    if ph == 13:
                        rc = lib.kaon_momentum_sumsq(ctypes.byref(plan.launch), ctypes.byref(h), s)
                    else:
                        rc = lib.kaon_msam_apply(ctypes.byref(plan.launch), ctypes.byref(h), f, float("inf"), 2, s)
                    _lib.check(rc, "msam pass")
                    e1.record()
                    torch.cuda.synchronize()
                    acc = out.setdefault(ph, [0.0] * reps)
                    acc[r] += e0.elapsed_time(e1)
    return {ph: sum(v) / len(v) for ph, v in out.items()}


def _cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it: the model string, with its family /
    model / stepping numbers, the microcode revision and the logical CPU count (a
    virtualized host may report only a short model name)."""
    info: dict[str, str] = {}
    n = 0
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if ":" not in line:
                    continue
                k, v = (s.strip() for s in line.split(":", 1))
                if k == "processor":
                    n += 1
                info.setdefault(k, v)
    except OSError:
        return "unknown"
    name = info.get("model name", "unknown")
    detail = ", ".join(f"{k} {info[k]}" for k in ("cpu family", "model", "stepping", "microcode") if k in info)
    return f"{name} ({detail}; {n} logical CPUs)" if detail else f"{name} ({n} logical CPUs)"


def cpu_baseline(params, name, budget_s: float) -> dict:
    """The CPU oracle (oracle/kaon_oracle.c, the C restatement of the reference's
    per-element step) over the same tensors on the host's cores: one oracle
    optimizer per tensor, the tensors spread over a thread pool (the C calls run
    outside the GIL), one warmup step, then the median of three timed steps.
    The whole set is timed when a step fits the budget; otherwise the largest
    prefix of a fixed random order of the tensors that does."""
    import statistics
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np
    import torch

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    w = WORKLOADS[name]
    kw = w["kw"]
    group = dict(lr=kw["lr"], betas=kw["betas"], eps=(1e-30, 1e-3), weight_decay=0.1 if w["opt"] == "nekaon" else 0.0,
                 clip_threshold=1.0, momentum_dtype=kw["momentum_dtype"],
                 momentum_4bit_block=kw.get("momentum_4bit_block", 128), cautious=True,
                 gradient_centralization=w["opt"] != "adamuon", bf16_method="stochastic_rounding", k=1.5,
                 ns_steps=kw.get("ns_steps", 2))
    if w["opt"] == "adapnm":
        group.update(eps=1e-8, beta0=kw["beta0"], ams_bound=False)
    if w["opt"] == "msam":
        group.update(rho=kw["rho"], norm="global", msam_eps=1e-12)
    if w["opt"] == "kprodigy":
        group.update(beta3=None, eps=1e-8, decouple=True, use_bias_correction=False, safeguard_warmup=False,
                     d=1e-6, d0=1e-6, d_max=1e-6, d_numerator=0.0, d_coef=1.0, growth_rate=float("inf"),
                     d_update_freq=1, slice_p=kw.get("slice_p", 1), k=0,
                     second_moment=kw.get("second_moment", "full"), eps_factored=1e-30, cautious=False,
                     factor_conv_as_matrix=True)
    order = [int(i) for i in np.random.default_rng(0).permutation(len(params))]
    if w["opt"] == "adamuon":
        # the oracle's scalar GEMMs take minutes on a 1280 x 11520 matrix: the
        # matrices with min(R, C) <= 640 (and the 1-D params)
        order = [i for i in order if params[i].ndim < 2 or min(params[i].shape[0],
                                                               params[i].numel() // params[i].shape[0]) <= 640]
    threads = min(_cpu_threads(), 16)
    oopt_name = "adakaon" if w["opt"] == "nekaon" else ("adakaon" if w["opt"] == "msam" else w["opt"])

    def build(i):
        p = params[i]
        prm = O.OParam(p=p.detach().view(torch.int16).cpu().numpy().view(np.uint16).copy(), p_dtype=O.BF16,
                       shape=tuple(p.shape), tensor_id=i,
                       g=p.grad.view(torch.int16).cpu().numpy().view(np.uint16).copy(), g_dtype=O.BF16)
        return O.OracleOptimizer([prm], oopt_name, group, seed=0), prm.numel

    with ThreadPoolExecutor(threads) as pool:
        # warmup on the whole candidate set, timed per tensor to size the timed set
        opts, sizes, secs = [], [], []
        t_all = 0.0
        for i in order:
            o, n = build(i)
            opts.append(o)
            sizes.append(n)
        def step_one(o):
            t = time.perf_counter()
            o.step()
            return time.perf_counter() - t
        t0 = time.perf_counter()
        secs = list(pool.map(step_one, opts))
        warm = time.perf_counter() - t0
        # the timed set: everything if a step fits the budget, else a prefix of the order
        k = len(opts)
        if warm > budget_s:
            acc, k = 0.0, 0
            for s_ in secs:
                if acc + s_ / threads > budget_s:
                    break
                acc += s_ / threads
                k += 1
            k = max(k, 1)
        timed = opts[:k]
        nparam = sum(sizes[:k])
        walls = []
        for _ in range(3):
            t0 = time.perf_counter()
            list(pool.map(lambda o: o.step(), timed))
            walls.append(time.perf_counter() - t0)
    med = statistics.median(walls)
    what = "the whole set" if k == len(order) and w["opt"] != "adamuon" else f"{k} of the tensors"
    return {"value": nparam / med / 1e9, "unit": "Gparam/s", "cores": threads, "kind": "port",
            "cpu_model": _cpu_model(),
            "sample": f"one {w['opt']} step of {what} ({k} tensors, {nparam / 1e6:.1f}M params"
                      f"{'; matrices with min(R, C) <= 640' if w['opt'] == 'adamuon' else ''}), CPU oracle "
                      f"oracle/kaon_oracle.c over {threads} threads (one oracle optimizer per tensor), "
                      f"median of 3 steps after 1 warmup: {med:.2f} s/step (warmup {warm:.1f} s)",
            "steps_s": [round(x, 3) for x in walls]}


def torch_order_leg(params, name, steps: int = 5, warmup: int = 2) -> dict:
    """The workload's step with reduction_order="torch" (the fp32 sums in torch CPU's order,
    the reference's bits) on the same params and grads, a fresh optimizer: ms per step
    (HIP events) and the phase kernels' times."""
    import torch
    from kaon_amd import Adakaon, Lion

    w = WORKLOADS[name]
    cls = Adakaon if w["opt"] == "adakaon" else Lion
    opt = cls(params, reduction_order="torch", **w["kw"])
    for _ in range(warmup):
        opt.step()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        opt.step()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    nparam = sum(p.numel() for p in params)
    br = phase_breakdown(opt, name)
    del opt
    torch.cuda.empty_cache()
    return {"ms_per_step": round(ms, 4), "gparam_s": round(nparam / (ms * 1e-3) / 1e9, 2), "steps": steps,
            "phases_ms": {PHASE_NAMES[k]: round(v, 4) for k, v in sorted(br.items())},
            "note": "reduction_order='torch': GC / row / column / row-factor means as torch CPU's cascades and "
                    "the clip norm as its 8 sequential fma chains per tensor (phase 3 writes the divisor)"}


def _cpu_threads() -> int:
    """The host's cores for the CPU baselines: the process's affinity set, capped by the
    OMP_NUM_THREADS share the host gives the job when it sets one."""
    n = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS")
    return max(1, min(n, int(cap))) if cap and cap.isdigit() else max(1, n)


def cpu_torch_foreach(params, name, stride: int) -> dict:
    """The reference's CPU path: oracle/torch_foreach.py, a torch-CPU restatement of its
    native foreach step (GC batched by shape, the CPU stack budget min(64M, 4 * 2M),
    shape buckets, per-param steps above 2M elements, torch.randint SR draws), pinned
    bit for bit against the reference's fixtures by tests/test_torch_foreach_cpu.py.
    Every ``stride``-th tensor of a fixed random order of the set (1 = the whole
    set), its weights and grads copied to the host; one warmup step, then the median
    of three timed steps on all the job's host cores."""
    import statistics

    import numpy as np
    import torch

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import torch_foreach as TF

    w = WORKLOADS[name]
    kw = w["kw"]
    threads = _cpu_threads()
    torch.set_num_threads(threads)
    order = [int(i) for i in np.random.default_rng(0).permutation(len(params))][::stride]
    ps = [params[i].detach().cpu() for i in order]
    gs = [params[i].grad.detach().cpu() for i in order]
    nparam = sum(p.numel() for p in ps)
    group = dict(lr=kw["lr"], betas=kw["betas"], eps=(1e-30, 1e-3), weight_decay=0.0, clip_threshold=1.0,
                 momentum_dtype=kw["momentum_dtype"], cautious=True, gradient_centralization=True,
                 bf16_method="stochastic_rounding")
    cls = TF.ForeachAdakaon if w["opt"] == "adakaon" else TF.ForeachLion
    opt = cls(ps, [g.clone() for g in gs], group)
    t0 = time.perf_counter()
    opt.step()
    warm = time.perf_counter() - t0
    walls = []
    for _ in range(3):
        opt.gs[:] = [g.clone() for g in gs]  # each step centralizes its grads in place, as the reference does
        t0 = time.perf_counter()
        opt.step()
        walls.append(time.perf_counter() - t0)
    med = statistics.median(walls)
    nth = {2: "2nd", 3: "3rd"}.get(stride, f"{stride}th")
    what = "the whole set" if stride == 1 else f"every {nth} tensor of a fixed random order of the set"
    return {"value": round(nparam / med / 1e9, 4), "unit": "Gparam/s", "cores": threads, "kind": "port",
            "cpu_model": _cpu_model(), "ms_per_step": round(med * 1e3, 1),
            "full_set_s_per_step_est": round(med * sum(p.numel() for p in params) / nparam, 2),
            "sample": f"one {w['opt']} step (torch CPU, the reference's native foreach path restated in "
                      f"oracle/torch_foreach.py) over {what}: {len(ps)} tensors, {nparam / 1e6:.1f}M params; "
                      f"torch.set_num_threads({threads}); median of 3 steps after 1 warmup: {med:.2f} s/step "
                      f"(warmup {warm:.1f} s)",
            "steps_s": [round(x, 3) for x in walls]}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="adakaon_int8", choices=sorted(WORKLOADS))
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="time budget of one CPU-baseline step (the whole set is timed when it fits)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-stride", type=int, default=2,
                    help="the torch-CPU baseline (Adakaon / Lion workloads) times every N-th tensor of a fixed "
                         "order of the set (the default 2: half the set, ≈20 s of CPU work); 1 = the whole set")
    ap.add_argument("--no-breakdown", action="store_true")
    ap.add_argument("--no-torch-order", action="store_true",
                    help="skip the reduction_order='torch' timing of Adakaon / Lion workloads")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}, WORLD_SIZE {world}); "
              "the step shards by whole tensors with no exchange inside it, so N GPUs would run this same "
              "kernel on 1/N of the set", file=sys.stderr)
        return 2

    import torch
    from kaon_amd import workloads

    dev = torch.device("cuda:0")
    w = WORKLOADS[args.workload]
    shapes = w.get("shapes") or workloads.sdxl_shapes()
    pdt = torch.float32 if w.get("pdtype") == "f32" else torch.bfloat16
    nparam = workloads.n_params(shapes)
    print(f"[bench] {args.workload}: {len(shapes)} tensors, {nparam / 1e9:.3f}B params", file=sys.stderr, flush=True)
    params = workloads.make_params(shapes, dev, seed=0, dtype=pdt, outlier_frac=w.get("outliers", 0.0))
    opt = make_opt(args.workload, params)
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        opt.step()
    torch.cuda.synchronize()
    print("[bench] warmup done", file=sys.stderr, flush=True)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    t0.record()
    for _ in range(args.steps):
        opt.step()
    t1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms = t0.elapsed_time(t1) / args.steps
    gps = nparam / (ms * 1e-3) / 1e9
    bm = w["bm"]
    eb = 4.0 if pdt == torch.float32 else 2.0   # param and grad element bytes
    # a step that leaves p.grad centralized writes those gradients once more: eb bytes
    # per written element, averaged over the set
    gcw = gc_written_elems(opt, args.workload) / nparam
    b_alg = eb + 2.0 * eb + 2.0 * bm + w.get("b_neg", 0.0) + w.get("b_extra", 0.0) + eb * gcw
    step_gbs = b_alg * nparam / (ms * 1e-3) / 1e9
    print(f"[bench] {ms:.3f} ms/step, {gps:.1f} Gparam/s (wall {wall / args.steps * 1e3:.3f} ms/step)",
          file=sys.stderr, flush=True)

    if "shapes" in w:
        # a launch-bound configuration: the step time is the metric
        out = {"metric": LORA_METRIC, "value": round(ms, 4), "unit": "ms", "n_gpus": 1, "steps": args.steps,
               "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak",
               "vs_baseline": None, "dtype": "f32", "data": "synthetic",
               "config": {"workload": w["desc"], "n_tensors": len(shapes), "n_params": nparam, "params": "f32",
                          "grads": "f32", "momentum": w["kw"]["momentum_dtype"], "parallelism": "none (1 GPU)",
                          "wall_ms_per_step": round(wall / args.steps * 1e3, 4),
                          "launches_per_step": "5 kernels"}}
        if not args.no_breakdown:
            out["phases_ms"] = {PHASE_NAMES[k]: round(v, 4) for k, v in sorted(phase_breakdown(opt, args.workload)
                                                                                 .items())}
        print(json.dumps(out), flush=True)
        return 0
    ceiling = copy_ceiling_gbs(dev)
    mix = apply_mix_ceiling_gbs(dev)
    out = {
        "metric": METRIC, "value": round(gps, 2), "unit": "Gparam/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": w["desc"], "shape_set": "SDXL-UNet-shaped (1678 tensors)", "n_params": nparam,
                   "params": "bf16", "grads": "bf16",
                   "momentum": w["kw"]["momentum_dtype"] + (" x2 (m_pos, m_neg)" if w["opt"] == "adapnm" else ""),
                   "parallelism": "none (1 GPU)"},
        "step_roofline": {"bound": "hbm", "bytes_per_param": b_alg, "achieved": round(step_gbs, 1),
                          "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(step_gbs / HBM_PEAK_GBS, 4),
                          "copy_ceiling": round(ceiling, 1), "frac_of_copy": round(step_gbs / ceiling, 4),
                          "apply_mix_ceiling": round(mix, 1), "frac_of_apply_mix": round(step_gbs / mix, 4)},
    }
    if not args.no_breakdown:
        br = phase_breakdown(opt, args.workload)
        wd = w["opt"] == "nekaon"
        dom = max(br, key=lambda k: br[k])
        if dom == 9:
            fl = ns_flops(shapes, w["kw"]["ns_steps"])
            ach = fl / (br[dom] * 1e-3) / 1e12
            out["roofline"] = {"bound": "mfma", "achieved": round(ach, 1), "peak": BF16_MFMA_PEAK_TFLOPS,
                               "unit": "TFLOP/s", "frac": round(ach / BF16_MFMA_PEAK_TFLOPS, 4),
                               "traffic": measured_traffic(args.workload, dom),
                               "kernel": "phase 9 (newton_schulz: bf16 MFMA GEMMs)", "flops_per_launch": fl,
                               "avg_ms": round(br[dom], 4), "source": kernel_source_hash()}
            out["ns_library"] = ns_library_ms(dev, shapes, w["kw"]["ns_steps"])
        else:
            bpp = phase_bytes(dom, bm, wd, w["opt"], w) + (eb * gcw if dom == 6 else 0.0)
            ach = bpp * nparam / (br[dom] * 1e-3) / 1e9 if bpp else 0.0
            out["roofline"] = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                               "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": measured_traffic(args.workload, dom),
                               "kernel": f"phase {dom} ({PHASE_NAMES[dom]})", "bytes_per_param": bpp,
                               "avg_ms": round(br[dom], 4), "frac_of_apply_mix": round(ach / mix, 4),
                               "source": kernel_source_hash()}
        out["phases_ms"] = {PHASE_NAMES[k]: round(v, 4) for k, v in sorted(br.items())}
    if w["opt"] in ("adakaon", "lion") and not args.no_torch_order:
        out["torch_order"] = torch_order_leg(params, args.workload)
    if args.workload == "adakaon_int8" and not args.no_breakdown:
        # the launch-bound regime beside the headline (reference: 0.24 ms for its fused Adakaon
        # on this bag, benchmarks/control/RANKINGS.md:83, on its own hardware)
        out["lora_bag"] = {"ms_per_step": round(lora_bag_ms(dev), 4), "unit": "ms", "config": WORKLOADS["lora_bag"]["desc"]}
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        del opt
        if w["opt"] in ("adakaon", "lion") and w["kw"]["momentum_dtype"] != "4bit":
            # the reference's own CPU path (torch foreach), and the C oracle beside it
            out["cpu_baseline"] = cpu_torch_foreach(params, args.workload, args.cpu_stride)
            out["cpu_oracle_baseline"] = cpu_baseline(params, args.workload, args.cpu_seconds)
        else:
            out["cpu_baseline"] = cpu_baseline(params, args.workload, args.cpu_seconds)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
