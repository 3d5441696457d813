"""Write the fixtures that show the reference resuming from a kaon_amd checkpoint.

Run in the build container only (the reference is not present on the GPU box):

    python tests/golden/make_interop.py /root/reference/src [case ...]

For each case the oracle (the CPU restatement the HIP step matches bit for
bit) takes the case's first ``steps - 1`` steps.  Its weights and state are
put into a kaon_amd optimizer built over CPU tensors, and that optimizer's own
``state_dict()`` is the checkpoint: the code that writes it on the GPU.  The
checkpoint goes through ``torch.save`` / ``torch.load(weights_only=True)`` into
the reference optimizer's ``load_state_dict`` (src/kaon/adakaon.py:744-753,
src/kaon/_momentum_codec.py:417-452), which then takes the case's last step
with the oracle's Philox noise injected at its SR call sites (the hooks of
make_golden.py).  The fixture ``interop_<case>.npz`` holds the checkpoint's
tensors (``c{i}_*``, ``cp{i}``) and the reference's weights and state after
that step (``p{i}``, ``s{i}_*``).

tests/test_checkpoint_cpu.py replays the last step in the oracle from the
fixture's checkpoint; tests/test_gpu_checkpoint.py checks that the HIP
optimizer's state_dict after the first steps is that checkpoint, byte for byte.
"""
from __future__ import annotations

import io
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "oracle"))
sys.path.insert(0, os.path.join(REPO, "k-optimizers_amd"))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, HERE)

import oracle as O  # noqa: E402
from cases import CASES, grad_values  # noqa: E402
from golden_compare import build_oracle, set_grads  # noqa: E402
import make_golden as MG  # noqa: E402

torch.set_num_threads(1)

# Adakaon and Lion with each momentum codec and write method the resume tests cover
INTEROP_CASES = ("ada_int8_sr", "ada_4bit_sr", "ada_bf16_rn", "ada_kahan", "lion_int8_sr", "lion_4bit_rn")


def _tensor_of(a: np.ndarray, like: torch.Tensor) -> torch.Tensor:
    """The oracle's array as a tensor of ``like``'s dtype and shape (bf16 as bits)."""
    a = np.ascontiguousarray(a)
    if like.dtype == torch.bfloat16:
        t = torch.from_numpy(a.reshape(-1).view(np.int16).copy()).view(torch.bfloat16)
    else:
        t = torch.from_numpy(a.reshape(-1).astype(a.dtype, copy=True)).to(like.dtype)
    return t.reshape(like.shape)


def kaon_amd_checkpoint(case, oparams, steps_done: int) -> dict:
    """kaon_amd's state_dict with the oracle's weights and state, written by
    kaon_amd's own state_dict() over CPU tensors."""
    from gpu_cases import make_opt, tdtype

    pdt = tdtype(case["p_dtype"])
    params = []
    for prm in oparams:
        params.append(torch.nn.Parameter(_tensor_of(prm.p, torch.empty(prm.shape, dtype=pdt))))
    gdt = tdtype(case["g_dtype"])
    for p in params:
        p.grad = torch.zeros(p.shape, dtype=gdt)  # _init_state reads the grad's shape
    opt = make_opt(case, params)
    for g in opt.param_groups:
        for p in g["params"]:
            opt._init_state(p, opt.state[p], g)
    for p in params:
        p.grad = None
    for prm, p in zip(oparams, params):
        st = opt.state[p]
        for k, v in prm.state.items():
            if k.startswith("_"):
                continue
            if torch.is_tensor(st.get(k)):
                st[k] = _tensor_of(np.asarray(v), st[k])
            else:
                st[k] = type(st[k])(v) if k in st else v
    opt._t = steps_done
    return opt.state_dict(), params


def run(ref_kaon, name: str) -> dict:
    case = CASES[name]
    S = case["steps"]
    oparams, oopt = build_oracle(case)
    for step in range(1, S):
        set_grads(case, oparams, step)
        oopt.step()
    sd, cparams = kaon_amd_checkpoint(case, oparams, S - 1)
    buf = io.BytesIO()
    torch.save(sd, buf)
    buf.seek(0)
    loaded = torch.load(buf, weights_only=True)

    # the reference optimizer over the checkpoint's weights
    rparams = [torch.nn.Parameter(p.detach().clone()) for p in cparams]
    ropt = MG.make_opt(ref_kaon, case, rparams)
    ropt.load_state_dict(loaded)
    MG._CTX["seed"] = case["seed"]
    MG._CTX["ids"] = {p.data_ptr(): i for i, p in enumerate(rparams)}
    MG._CTX["step"] = S
    gdt = torch.bfloat16 if case["g_dtype"] == "bf16" else torch.float32
    for i, p in enumerate(rparams):
        p.grad = torch.from_numpy(grad_values(case, i, S)).to(gdt)
    ropt.step()

    out = {}
    for i, p in enumerate(cparams):
        out[f"cp{i}"] = MG._bits(p)
        for k, v in sd["state"][i].items():
            out[f"c{i}_{k}"] = MG._bits(v) if torch.is_tensor(v) else np.asarray(v)
    out["c_step"] = np.asarray(sd["kaon_amd"]["step"])
    out["c_sr_seed"] = np.asarray(sd["kaon_amd"]["sr_seed"])
    for i, p in enumerate(rparams):
        out[f"p{i}"] = MG._bits(p)
        for k, v in ropt.state[p].items():
            out[f"s{i}_{k}"] = MG._bits(v) if torch.is_tensor(v) else np.asarray(v)
    return out


def main() -> None:
    ref_src = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src"
    only = set(sys.argv[2:])
    sys.path.insert(0, ref_src)
    import kaon  # the reference package (this container only)

    MG._install_noise_hooks(kaon)
    for name in INTEROP_CASES:
        if only and name not in only:
            continue
        out = run(kaon, name)
        np.savez_compressed(os.path.join(HERE, f"interop_{name}.npz"), **out)
        print(name, "written", flush=True)


if __name__ == "__main__":
    main()
