"""Write the golden fixtures that pin the oracle's whole-step composition.

Run in the build container only (the reference is not present on the GPU box):

    python tests/golden/make_golden.py /root/reference/src [case ...]

It imports the reference ``kaon`` package (pure Python + torch CPU) and steps
its Adakaon / Lion / AdaMuon / Nekaon / MSAM / AdaPNM / KProdigy on small seeded inputs.  The codecs, the
SR bit trick, the cautious rule and the Philox stream are pinned by closed
forms and known-answer tests elsewhere; what only the reference itself can pin
is the composition of torch-CPU ops (lerp/FMA placement, bf16-rounded GC,
clip, codec ordering), so that is what these fixtures record.

Stochastic rounding is made deterministic by injecting noise: the reference's
``add_stochastic_`` call sites are wrapped so that the ``torch.randint`` draw
inside ``_add_stochastic_bf16_`` (src/kaon/_stochastic_rounding.py:88-94)
returns the oracle's Philox noise for (seed, step, tensor id, stream, element).
The SR arithmetic itself is the reference's.  Per-param paths
(``foreach=False``) are used for SR cases so each draw covers one parameter;
RN (``bf16_method="none"``) cases also run the foreach path.

Fixtures hold inputs' seeds and shapes, the final state and weights (small
cases), or per-step hashes, a strided weight sample and the full factored
state.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "oracle"))
sys.path.insert(0, HERE)

import oracle as O  # noqa: E402
from cases import CASES, CFG0, grad_values, param_values  # noqa: E402

torch.set_num_threads(1)

_CTX = {"step": 0, "stream": 1, "tid": None, "ids": {}}


def _install_noise_hooks(kaon_mod) -> None:
    import kaon._backend as backend
    import kaon.msam as msam_mod
    import kaon._stochastic_rounding as srmod

    real_add = srmod.add_stochastic_
    real_randint = torch.randint

    def fake_randint(*args, **kw):
        size = kw.get("size")
        tid = _CTX["tid"]
        assert tid is not None, "randint outside an instrumented SR call"
        n = int(np.prod(size))
        noise = O.sr_noise(n, _CTX["seed"], _CTX["step"], tid, _CTX["stream"])
        return torch.from_numpy(noise.astype(np.int32)).reshape(size)

    def add_sr(target, source, alpha=1.0):
        tid = _CTX["ids"].get(target.data_ptr())
        _CTX["tid"] = tid
        torch.randint = fake_randint
        try:
            real_add(target, source, alpha)
        finally:
            torch.randint = real_randint
            _CTX["tid"] = None

    backend.add_stochastic_ = add_sr
    msam_mod.add_stochastic_ = add_sr

    real_apply = msam_mod.MSAM._apply

    def apply(self, sign):
        _CTX["stream"] = 0 if sign < 0 else 2
        try:
            real_apply(self, sign)
        finally:
            _CTX["stream"] = 1

    msam_mod.MSAM._apply = apply
    # The Triton fast path is GPU-only; make sure MSAM takes the torch path.
    msam_mod.MSAM._apply_fused_4bit = lambda self, sign: None


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    return t.numpy().copy()


def build_params(case):
    params = []
    for i, shape in enumerate(case["shapes"]):
        v = param_values(case, i)
        dt = {"bf16": torch.bfloat16, "f16": torch.float16}.get(case["p_dtype"], torch.float32)
        params.append(torch.nn.Parameter(torch.from_numpy(v).to(dt)))
    return params


def make_opt(kaon, case, params):
    kw = dict(case["kwargs"])
    name = case["opt"]
    if name == "adakaon":
        return kaon.Adakaon(params, **kw)
    if name == "lion":
        return kaon.Lion(params, **kw)
    if name == "adamuon":
        return kaon.AdaMuon(params, **kw)
    if name == "nekaon":
        return kaon.Nekaon(params, **kw)
    if name == "adapnm":
        return kaon.AdaPNM(params, **kw)
    if name == "kprodigy":
        return kaon.KProdigy(params, **kw)
    if name == "msam":
        return kaon.MSAM(params, **kw)
    raise ValueError(name)


def name_of(case) -> str:
    return case["opt"]


def run_case(kaon, case):
    params = build_params(case)
    opt = make_opt(kaon, case, params)
    _CTX["seed"] = case["seed"]
    _CTX["ids"] = {p.data_ptr(): i for i, p in enumerate(params)}
    hashes = []
    d_traj = []
    mnorm_traj = []
    out_steps = {}
    for step in range(1, case["steps"] + 1):
        for i, p in enumerate(params):
            g = grad_values(case, i, step)
            gdt = {"bf16": torch.bfloat16, "f16": torch.float16}.get(case["g_dtype"], torch.float32)
            p.grad = torch.from_numpy(g).to(gdt)
        _CTX["step"] = step
        opt.step()
        if name_of(case) == "kprodigy":
            d_traj.append(opt.param_groups[0]["d"])
        if name_of(case) == "msam":
            mnorm_traj.append(opt._mnorm)
            for i, p in enumerate(params):  # the momentum the norm was taken over
                for k in ("m", "m_scale"):
                    if k in opt.inner.state[p]:
                        out_steps[f"t{step}_s{i}_{k}"] = _bits(opt.inner.state[p][k])
        if step == 1 and case.get("sample_stride"):
            step1 = [_bits(p).reshape(-1)[::case["sample_stride"]] for p in params]
        hashes.append(hashlib.sha256(b"".join(_bits(p).tobytes() for p in params)).hexdigest())
    if case.get("eval_train"):
        _CTX["step"] = case["steps"]
        opt.eval()
        eval_p = [_bits(p) for p in params]
        opt.train()
    out = {"hashes": hashes}
    if name_of(case) == "kprodigy":
        # the group's D state (kprodigy.py:365-380): d after every step, and the final scalars
        grp = opt.param_groups[0]
        out["d_traj"] = np.array(d_traj, dtype=np.float64)
        for key in ("d", "d_max", "d_numerator"):
            out[f"g_{key}"] = np.array(grp[key], dtype=np.float64)
        out["g_k"] = np.array(grp["k"], dtype=np.int64)
    if name_of(case) == "msam":
        # MSAM's cached ||m|| after every step (msam.py:191-199, 395-397)
        out["mnorm_traj"] = np.array(mnorm_traj, dtype=np.float64)
        out.update(out_steps)
    inner = getattr(opt, "inner", opt)
    for i, p in enumerate(params):
        st = inner.state[p]
        pb = _bits(p)
        if case.get("sample_stride"):
            s = case["sample_stride"]
            out[f"p{i}_sample"] = pb.reshape(-1)[::s]
            out[f"p{i}_step1_sample"] = step1[i]
        else:
            out[f"p{i}"] = pb
        for k, v in st.items():
            if torch.is_tensor(v):
                out[f"s{i}_{k}"] = _bits(v)
            else:
                out[f"s{i}_{k}"] = np.asarray(v)
        if case.get("eval_train"):
            out[f"p{i}_eval"] = eval_p[i]
    return out


def main() -> None:
    """argv: [reference src dir] [case names ...]; no names = every case."""
    ref_src = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src"
    only = set(sys.argv[2:])
    sys.path.insert(0, ref_src)
    import kaon  # the reference package (this container only)

    _install_noise_hooks(kaon)
    meta = {"torch": torch.__version__, "cpu_capability": torch.backends.cpu.get_cpu_capability(),
            "threads": torch.get_num_threads(), "kaon_version": kaon.__version__, "cases": {}}
    meta_path = os.path.join(HERE, "golden_meta.json")
    if only and os.path.exists(meta_path):
        with open(meta_path) as fh:
            meta["cases"] = json.load(fh).get("cases", {})
    for name, case in list(CASES.items()) + [("cfg0", CFG0)]:
        if only and name not in only:
            continue
        out = run_case(kaon, case)
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **{k: v for k, v in out.items() if k != "hashes"})
        meta["cases"][name] = {"hashes": out["hashes"]}
        print(name, out["hashes"][-1][:16], flush=True)
    with open(meta_path, "w") as fh:
        json.dump(meta, fh, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
