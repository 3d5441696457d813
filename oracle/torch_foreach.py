"""torch-CPU restatement of the reference's native *foreach* step.

Test and measurement infrastructure, not the product: bench.py's cpu_baseline
leg times it on the host's cores, and tests/test_torch_foreach_cpu.py pins it
against the reference's own fixtures.  It is the reference's CPU path --
the same torch ops in the same order, the same shape buckets, the same stack
budget, the same per-param branch -- so its time is what the reference takes
on the same host.  The product path never imports it.

Adakaon (src/kaon/adakaon.py):
* GC first, batched by grad shape (centralize_grads_, _backend.py:147-177);
* routing (_native_dispatch, :357-383): the stack budget on a CPU device is
  min(64M, 4 * foreach_batch_cutoff) elements (foreach_budget,
  _backend.py:59-77); a param joins the foreach path if it has ndim >= 1, at
  most min(cutoff, budget // 2) elements and is contiguous (:754-791), and the
  group does when its clip is on and it does not write by kahan (:748-758);
  with fewer than two eligible params everything steps per param;
* _step_foreach (:793-838): factored buckets keyed by (matrixized shape, dtype,
  matrixize) in chunks of budget // (R * C) params, 1-D buckets keyed by length;
* _factored_bucket (:840-906), _nonfactored_bucket (:908-966),
  _step_one_param (:968-1014);
* codecs (_momentum_codec.py): float storage lerps in its own dtype
  (:253-290); int8 dequantizes with the per-row scale, lerps in fp32 and
  requantizes (:293-339);
* cautious_batched_ / cautious_one_ (_backend.py:127-142); subtract_batched_ /
  subtract_one_ (:82-122); add_stochastic_ (_stochastic_rounding.py:39-103),
  whose torch.randint draw a caller may replace (``randint``) to inject noise.

Lion (src/kaon/lion.py:322-485): the same GC and routing, buckets keyed by
exact shape and flattened to [N, L], the stacked int8 requant per param row.

Codecs restated: float32, bfloat16 and int8 (the baseline's workloads use
int8; 4-bit workloads keep the C oracle as their baseline).
"""
from __future__ import annotations

import math
from typing import Any, Callable

import torch

FOREACH_BATCH_CUTOFF = 2_000_000   # _backend.py:53
CPU_STACK_ELEMS = 64_000_000       # _backend.py:56, the budget off a GPU


def cpu_stack_budget(cutoff: int = FOREACH_BATCH_CUTOFF) -> int:
    """foreach_budget on a CPU device (_backend.py:59-77): min(64M, 4 * cutoff)."""
    return min(CPU_STACK_ELEMS, 4 * cutoff)


# ------------------------------------------------------------------ shared ops
def centralize_(grads: list[torch.Tensor]) -> None:
    """GC of every grad with ndim >= 2: minus its mean over the fan-in dims, in the grad's
    dtype; same-shape grads stacked and centralized together, lone shapes in place."""
    by_shape: dict[tuple, list[torch.Tensor]] = {}
    for g in grads:
        if g.ndim >= 2:
            by_shape.setdefault(tuple(g.shape), []).append(g)
    for gl in by_shape.values():
        if len(gl) == 1:
            g = gl[0]
            g.sub_(g.mean(dim=tuple(range(1, g.ndim)), keepdim=True))
        else:
            st = torch.stack(gl)
            st.sub_(st.mean(dim=tuple(range(2, st.ndim)), keepdim=True))
            torch._foreach_copy_(gl, list(st.unbind(0)))


def sr_add_(target: torch.Tensor, source: torch.Tensor, alpha: float, randint: Callable) -> None:
    """target += alpha * source, stochastically rounded to bf16 by the int32 bit trick
    (noise in [0, 2^16) added to the fp32 bits, low half cleared); fp32 targets add."""
    if target.dtype == torch.float32:
        target.add_(source, alpha=alpha)
        return
    x = target.float()
    x.add_(source if source.dtype == torch.float32 else source.float(), alpha=alpha)
    bits = x.view(torch.int32)
    bits.add_(randint(0, 0x10000, size=bits.shape, dtype=torch.int32)).bitwise_and_(-0x10000)
    target.copy_(x.to(torch.bfloat16))


def subtract_one_(p: torch.Tensor, delta: torch.Tensor, st: dict, method: str, randint: Callable) -> None:
    low = p.dtype in (torch.bfloat16, torch.float16)
    if low and method == "kahan":
        shift = st["shift"]
        shift.sub_(delta.to(p.dtype))
        before = p.clone()
        p.add_(shift)
        shift.add_(before.sub_(p))
    elif low and method == "stochastic_rounding" and p.dtype == torch.bfloat16:
        sr_add_(p, delta, -1.0, randint)
    else:
        p.sub_(delta.to(p.dtype))


def subtract_stacked_(views: list[torch.Tensor], delta: torch.Tensor, method: str, randint: Callable) -> None:
    if views[0].dtype == torch.bfloat16 and method == "stochastic_rounding":
        w = torch.stack(views)
        sr_add_(w, delta, -1.0, randint)
        torch._foreach_copy_(views, list(w.unbind(0)))
    elif views[0].dtype == delta.dtype:
        torch._foreach_sub_(views, list(delta.unbind(0)))
    else:
        torch._foreach_sub_(views, [d.to(views[0].dtype) for d in delta.unbind(0)])


def cautious_stacked_(delta: torch.Tensor, grad: torch.Tensor) -> torch.Tensor:
    keep = (delta * grad > 0).to(delta.dtype)
    n = delta.shape[0]
    den = keep.reshape(n, -1).mean(dim=1).clamp_(min=1e-8).view(n, *([1] * (delta.ndim - 1)))
    return delta.mul_(keep).div_(den)


def cautious_one_(delta: torch.Tensor, grad: torch.Tensor) -> torch.Tensor:
    keep = (delta * grad > 0).to(delta.dtype)
    return delta.mul_(keep).div_(keep.mean().clamp_(min=1e-8))


def quant_int8_rows(m: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """int8 codes and scales over the last axis: absmax / 127 (floor 1e-12), RNE codes."""
    scale = m.abs().amax(dim=-1, keepdim=True).clamp_(min=1e-12) / 127.0
    return (m / scale).round_().clamp_(-127, 127).to(torch.int8), scale


def quant_int8_param(m: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-param int8 requant: per-row (dim 0) scale for ndim >= 2, one scalar for 1-D."""
    dims = tuple(range(1, m.ndim)) if m.ndim >= 2 else ()
    scale = m.abs().amax(dim=dims, keepdim=True).clamp_(min=1e-12) / 127.0
    return (m / scale).round_().clamp_(-127, 127).to(torch.int8), scale


def init_momentum(st: dict, g: torch.Tensor, md: str) -> None:
    if md in ("bfloat16", "float32"):
        st["m"] = torch.zeros_like(g, dtype=torch.bfloat16 if md == "bfloat16" else torch.float32)
    elif md == "int8":
        st["m"] = torch.zeros_like(g, dtype=torch.int8)
        st["m_scale"] = torch.ones((g.shape[0],) + (1,) * (g.ndim - 1) if g.ndim >= 2 else (),
                                   dtype=torch.float32)
    else:
        raise NotImplementedError(f"momentum_dtype {md!r} is not restated here")


class _Base:
    """Params as (weight, grad) tensor pairs on the CPU; state per param index."""

    def __init__(self, ps: list[torch.Tensor], gs: list[torch.Tensor], group: dict[str, Any],
                 cutoff: int = FOREACH_BATCH_CUTOFF, foreach: bool = True) -> None:
        self.ps, self.gs, self.group = ps, gs, dict(group)
        self.state: list[dict] = [{} for _ in ps]
        self.cutoff = cutoff
        self.foreach = foreach
        # the SR draw (torch.randint in the reference); ``writing`` lists the param indices
        # whose weights the current draw rounds, in stack order (a noise-injecting test reads it)
        self.randint: Callable = torch.randint
        self.writing: list[int] = []

    def _route(self, eligible_group: bool) -> tuple[list[int], list[int]]:
        idx = list(range(len(self.ps)))
        if not (self.foreach and eligible_group):
            return [], idx
        budget = cpu_stack_budget(self.cutoff)
        cut = min(self.cutoff, budget // 2)
        fast, slow = [], []
        for i in idx:
            (fast if self._eligible(i, cut) else slow).append(i)
        if len(fast) < 2:
            return [], idx
        return fast, slow

    def _eligible(self, i: int, cut: int) -> bool:
        p, g = self.ps[i], self.gs[i]
        if p.ndim == 0 or p.numel() > cut:
            return False
        if self.group["bf16_method"] == "stochastic_rounding" and p.dtype == torch.float16:
            return False
        return p.ndim <= 2 or (p.is_contiguous() and g.is_contiguous())


class ForeachAdakaon(_Base):
    def step(self) -> None:
        g = self.group
        if g["gradient_centralization"]:
            centralize_(self.gs)
        fast, slow = self._route(g["clip_threshold"] > 0 and g["bf16_method"] != "kahan")
        if fast:
            self._foreach(fast)
        for i in slow:
            self._one(i)

    def _init(self, i: int) -> None:
        st, gr = self.state[i], self.gs[i]
        if st:
            return
        if gr.ndim >= 2:
            st["row"] = torch.zeros(gr.shape[0], dtype=torch.float32)
            st["col"] = torch.zeros(gr.numel() // gr.shape[0], dtype=torch.float32)
        else:
            st["v"] = torch.zeros_like(gr, dtype=torch.float32)
        if self.group["betas"][0] > 0:
            init_momentum(st, gr, self.group["momentum_dtype"])
        if self.ps[i].dtype in (torch.bfloat16, torch.float16) and self.group["bf16_method"] == "kahan":
            st["shift"] = torch.zeros_like(self.ps[i])

    def _foreach(self, idx: list[int]) -> None:
        budget = cpu_stack_budget(self.cutoff)
        fac: dict[tuple, list[int]] = {}
        flat: dict[tuple, list[int]] = {}
        for i in idx:
            self._init(i)
            gr = self.gs[i]
            if gr.ndim >= 2:
                mz = gr.ndim > 2
                eff = (gr.shape[0], gr.numel() // gr.shape[0]) if mz else tuple(gr.shape)
                fac.setdefault((eff, self.ps[i].dtype, mz), []).append(i)
            else:
                flat.setdefault((gr.shape[0], self.ps[i].dtype), []).append(i)
        for (eff, _dt, mz), il in fac.items():
            k = max(1, budget // max(eff[0] * eff[1], 1))
            for a in range(0, len(il), k):
                self._bucket(il[a:a + k], eff, mz)
        for (length, _dt), il in flat.items():
            k = max(1, budget // max(length, 1))
            for a in range(0, len(il), k):
                self._bucket(il[a:a + k], (length,), False)

    def _ema_stacked(self, il: list[int], upd: torch.Tensor, view: Callable, eff: tuple) -> torch.Tensor:
        md, b1 = self.group["momentum_dtype"], self.group["betas"][0]
        sts = [self.state[i] for i in il]
        if md in ("bfloat16", "float32"):
            ms = [view(s["m"]) for s in sts]
            mom = torch.stack(ms)
            mom.lerp_(upd.to(mom.dtype), 1.0 - b1)
            torch._foreach_copy_(ms, list(mom.unbind(0)))
            return mom.float()
        rs = (eff[0], 1) if len(eff) == 2 else (1,)
        sc = torch.stack([s["m_scale"].view(*rs) for s in sts])
        m = torch.stack([view(s["m"]) for s in sts]).float().mul_(sc)
        m.lerp_(upd, 1.0 - b1)
        delta = m.clone()
        q, nsc = quant_int8_rows(m)
        torch._foreach_copy_([view(s["m"]) for s in sts], list(q.unbind(0)))
        for s, x in zip(sts, nsc.unbind(0)):
            s["m_scale"].copy_(x.view_as(s["m_scale"]))
        return delta

    def _bucket(self, il: list[int], eff: tuple, mz: bool) -> None:
        g = self.group
        b1, b2 = g["betas"]
        eps1, lr, clip, wd = g["eps"][0], g["lr"], g["clip_threshold"], g["weight_decay"]
        n = len(il)
        factored = len(eff) == 2
        view = (lambda t: t.view(*eff)) if mz else (lambda t: t)
        grad = torch.stack([view(self.gs[i]).float() for i in il])
        gsq = grad * grad
        if eps1 > 0:
            gsq = gsq.add_(eps1)
        if factored:
            R, C = eff
            rows = [self.state[i]["row"] for i in il]
            cols = [self.state[i]["col"] for i in il]
            row, col = torch.stack(rows), torch.stack(cols)
            row.lerp_(gsq.mean(dim=-1), 1.0 - b2)
            col.lerp_(gsq.mean(dim=-2), 1.0 - b2)
            torch._foreach_copy_(rows, list(row.unbind(0)))
            torch._foreach_copy_(cols, list(col.unbind(0)))
            rf = row.div(row.mean(dim=-1, keepdim=True)).rsqrt_().unsqueeze(-1)
            upd = grad.mul(rf).mul_(col.rsqrt().unsqueeze(-2))
            rms = upd.reshape(n, -1).norm(2, dim=1) / math.sqrt(R * C)
            upd.div_(rms.div_(clip).clamp_(min=1.0).view(n, 1, 1))
        else:
            vs = [self.state[i]["v"] for i in il]
            v = torch.stack(vs)
            v.lerp_(gsq, 1.0 - b2)
            torch._foreach_copy_(vs, list(v.unbind(0)))
            upd = grad.mul(v.rsqrt())
            rms = upd.norm(2, dim=1) / math.sqrt(eff[0])
            upd.div_(rms.div_(clip).clamp_(min=1.0).view(n, 1))
        upd.mul_(lr)
        delta = self._ema_stacked(il, upd, view, eff) if b1 > 0 else upd
        if wd != 0:
            delta = delta.add_(torch.stack([view(self.ps[i]).float() for i in il]), alpha=lr * wd)
        if g["cautious"]:
            delta = cautious_stacked_(delta, grad)
        self.writing = il
        subtract_stacked_([view(self.ps[i]) for i in il], delta, g["bf16_method"], self.randint)

    def _one(self, i: int) -> None:
        g = self.group
        b1, b2 = g["betas"]
        eps1, lr, clip, wd = g["eps"][0], g["lr"], g["clip_threshold"], g["weight_decay"]
        self._init(i)
        st, p = self.state[i], self.ps[i]
        gf = self.gs[i] if self.gs[i].dtype == torch.float32 else self.gs[i].float()
        if gf.ndim >= 2:
            gv = gf.reshape(gf.shape[0], -1) if gf.ndim > 2 else gf
            gsq = gv.pow(2)
            if eps1 > 0:
                gsq.add_(eps1)
            st["row"].lerp_(gsq.mean(dim=-1), 1.0 - b2)
            st["col"].lerp_(gsq.mean(dim=-2), 1.0 - b2)
            rf = st["row"].div(st["row"].mean(dim=-1, keepdim=True)).rsqrt_().unsqueeze(-1)
            upd = gv.mul(rf).mul_(st["col"].rsqrt().unsqueeze(-2))
            if gf.ndim > 2:
                upd = upd.view_as(gf)
        else:
            gsq = gf * gf
            if eps1 > 0:
                gsq.add_(eps1)
            st["v"].lerp_(gsq, 1.0 - b2)
            upd = gf.mul(st["v"].rsqrt())
        if clip > 0:
            upd.div_((upd.norm(2) / math.sqrt(max(upd.numel(), 1)) / clip).clamp_(min=1.0))
        upd.mul_(lr)
        if b1 > 0:
            md = g["momentum_dtype"]
            if md in ("bfloat16", "float32"):
                m = st["m"]
                m.lerp_(upd.to(m.dtype), 1.0 - b1)
                delta = m.float() if m.dtype != torch.float32 else m.clone()
            else:
                m = st["m"].float() * st["m_scale"]
                m.lerp_(upd, 1.0 - b1)
                delta = m.clone()
                st["m"], st["m_scale"] = quant_int8_param(m)
        else:
            delta = upd
        if wd != 0:
            delta = delta.add_(p if p.dtype == torch.float32 else p.float(), alpha=lr * wd)
        if g["cautious"]:
            delta = cautious_one_(delta, gf)
        self.writing = [i]
        subtract_one_(p, delta, st, g["bf16_method"], self.randint)


class ForeachLion(_Base):
    def step(self) -> None:
        g = self.group
        if g["gradient_centralization"]:
            centralize_(self.gs)
        fast, slow = self._route(g["bf16_method"] != "kahan")
        if fast:
            budget = cpu_stack_budget(self.cutoff)
            buckets: dict[tuple, list[int]] = {}
            for i in fast:
                self._init(i)
                buckets.setdefault((tuple(self.ps[i].shape), self.ps[i].dtype), []).append(i)
            for (shape, _dt), il in buckets.items():
                length = math.prod(shape)
                k = max(1, budget // max(length, 1))
                for a in range(0, len(il), k):
                    self._bucket(il[a:a + k], shape, length)
        for i in slow:
            self._one(i)

    def _init(self, i: int) -> None:
        st = self.state[i]
        if st:
            return
        init_momentum(st, self.gs[i], self.group["momentum_dtype"])
        if self.ps[i].dtype in (torch.bfloat16, torch.float16) and self.group["bf16_method"] == "kahan":
            st["shift"] = torch.zeros_like(self.ps[i])

    def _bucket(self, il: list[int], shape: tuple, length: int) -> None:
        g = self.group
        b1, b2 = g["betas"]
        md = g["momentum_dtype"]
        n = len(il)
        sts = [self.state[i] for i in il]
        grad = torch.stack([self.gs[i].reshape(length).float() for i in il])
        row = shape[0] if len(shape) >= 2 else 1
        rest = max(length // row, 1)
        if md in ("bfloat16", "float32"):
            m = torch.stack([s["m"] for s in sts]).float().reshape(n, length)
        else:
            m = torch.stack([s["m"].reshape(row, rest) for s in sts]).float()
            m = m.mul_(torch.stack([s["m_scale"].reshape(row, 1) for s in sts])).reshape(n, length)
        delta = torch.sign(m.mul(b1).add_(grad, alpha=1.0 - b1))
        m.mul_(b2).add_(grad, alpha=1.0 - b2)
        if md in ("bfloat16", "float32"):
            torch._foreach_copy_([s["m"] for s in sts], list(m.reshape(n, *shape).unbind(0)))
        else:
            q, nsc = quant_int8_rows(m.reshape(n, row, rest))
            torch._foreach_copy_([s["m"].reshape(row, rest) for s in sts], list(q.unbind(0)))
            for s, x in zip(sts, nsc.unbind(0)):
                s["m_scale"] = x.reshape(row, 1) if len(shape) >= 2 else x.reshape(1)
        if g["weight_decay"] != 0:
            delta = delta.add_(torch.stack([self.ps[i].reshape(length).float() for i in il]),
                               alpha=g["weight_decay"])
        if g["cautious"]:
            delta = cautious_stacked_(delta, grad)
        delta.mul_(g["lr"])
        self.writing = il
        subtract_stacked_([self.ps[i].reshape(length) for i in il], delta, g["bf16_method"], self.randint)

    def _one(self, i: int) -> None:
        g = self.group
        b1, b2 = g["betas"]
        md = g["momentum_dtype"]
        self._init(i)
        st, p = self.state[i], self.ps[i]
        gf = self.gs[i] if self.gs[i].dtype == torch.float32 else self.gs[i].float()
        m = st["m"].float() if md in ("bfloat16", "float32") else st["m"].float().mul_(st["m_scale"])
        delta = torch.sign(m.mul(b1).add_(gf, alpha=1.0 - b1))
        m.mul_(b2).add_(gf, alpha=1.0 - b2)
        if md in ("bfloat16", "float32"):
            st["m"].copy_(m)
        else:
            st["m"], st["m_scale"] = quant_int8_param(m)
        if g["weight_decay"] != 0:
            delta = delta.add_(p if p.dtype == torch.float32 else p.float(), alpha=g["weight_decay"])
        if g["cautious"]:
            delta = cautious_one_(delta, gf)
        delta.mul_(g["lr"])
        self.writing = [i]
        subtract_one_(p, delta, st, g["bf16_method"], self.randint)


__all__ = ["CPU_STACK_ELEMS", "FOREACH_BATCH_CUTOFF", "ForeachAdakaon", "ForeachLion", "centralize_",
           "cpu_stack_budget"]
