"""MSAM (Momentum-SAM) over a kaon_amd optimizer on the MI355X HIP step.

Reference: src/kaon/msam.py:73-421.  Each step removes the previous climb,
runs the inner step at the true weights, and climbs along the refreshed
momentum for the next forward/backward:

* ``norm="global"`` (the default): ``e = rho * m / (||m|| + eps)`` with ``||m||``
  over every momentum of the net (``_global_mnorm``, :191-199) -- a
  cross-tensor reduction between the inner step and the climb
  (``kaon_momentum_sumsq``, the tensors added in param order in fp32);
* ``norm="tensor"``: ``e = rho * m / (||m|| + eps)`` with each tensor's own norm
  (:219-222), recomputed at every climb and removal (``kaon_momentum_sumsq`` then
  ``kaon_msam_apply_tensor``, which forms each tensor's scale on the device);
* ``norm="none"``: ``e = clamp(nan_to_num(rho * m), +-|rho| * clip * lr)`` with the
  bound frozen at climb time (:169-188, Nekaon's form).

Over a plain :class:`Adakaon` the removal (and for ``norm="none"`` the climb)
is folded into the Adakaon apply pass, as three stochastic roundings of one
register value (SR noise streams 0, 1, 2); over any other kaon_amd optimizer
with a momentum buffer they are separate ``kaon_msam_apply`` passes, as in the
reference; ``norm="tensor"`` always takes those separate passes.  As in the
reference, the global and tensor norms scale the momentum with no sanitizing
(a NaN or inf coordinate reaches the weights; a tensor whose norm is NaN goes
NaN whole), while ``norm="none"`` maps NaN to a zero climb and clamps +-inf.
"""
from __future__ import annotations

import ctypes
import math
from collections import defaultdict
from typing import Any, Iterable

import numpy as np
import torch

from . import _engine as E
from . import _lib as L
from .adakaon import Adakaon


def _ptr_or0(t: torch.Tensor | None) -> int:
    return t.data_ptr() if t is not None else 0


class MSAM(torch.optim.Optimizer):
    def __init__(
        self,
        params: Iterable[Any],
        base_optimizer: type | None = None,
        rho: float = 0.3,
        norm: str = "global",
        eps: float = 1e-12,
        **kwargs: Any,
    ) -> None:
        if eps < 0.0:
            raise ValueError(f"eps must be >= 0, got {eps}")
        if norm not in ("global", "tensor", "none"):
            raise ValueError(f"norm must be 'global', 'tensor' or 'none', got {norm!r}")
        base = Adakaon if base_optimizer is None else base_optimizer
        self._bind(base(params, **kwargs), rho, norm, eps)

    def _bind(self, inner: torch.optim.Optimizer, rho: float, norm: str, eps: float) -> None:
        """Wrap ``inner``: the param groups and defaults are its own; MSAM keeps no
        per-param state (torch.optim.Optimizer bookkeeping: hooks, LR schedulers)."""
        if not hasattr(inner, "_tensor_ids"):
            raise TypeError("kaon_amd: MSAM wraps a kaon_amd optimizer that owns the momentum "
                            f"(Adakaon, Lion, AdaMuon, AdaPNM, KProdigy), got {type(inner).__name__}")
        super().__init__([p for g in inner.param_groups for p in g["params"]], dict(inner.defaults))
        self.inner = inner
        self.base_optimizer = inner
        self.param_groups = self.inner.param_groups
        self.defaults = self.inner.defaults
        self.state = defaultdict(dict)   # no per-param state of its own
        self.rho = float(rho)
        self.norm = norm
        self.eps = float(eps)
        self._train_mode = True
        self._has_e = False
        self._mnorm = 0.0
        self._eclamp: dict[int, float] = {}
        self._fused = type(inner) is Adakaon
        self._mplans: dict[tuple, tuple[tuple, E.Plan, list[int], torch.Tensor]] = {}

    # ---------------------------------------------------------------- plans
    def _has_momentum(self) -> bool:
        return any("m" in self.inner.state.get(p, ())
                   for g in self.param_groups for p in g["params"])

    def _momentum_plans(self, gradless: bool = False) -> list[tuple[int, int, E.Plan, list[int], torch.Tensor]]:
        """(gid, p dtype, plan, param positions, stat word index) over the params with a
        momentum buffer (with ``gradless``: only those without a gradient now), cached
        while the param and state pointers hold."""
        tids = self.inner._tensor_ids()
        by_key: dict[tuple[int, int], list[torch.Tensor]] = {}
        for gid, group in enumerate(self.param_groups):
            for p in group["params"]:
                if gradless and p.grad is not None:
                    continue
                st = self.inner.state.get(p)
                if st and "m" in st:
                    by_key.setdefault((gid, E.dtype_code(p.dtype)), []).append(p)
        out = []
        for (gid, pdt), plist in by_key.items():
            ptrs = tuple((p.data_ptr(), self.inner.state[p]["m"].data_ptr(),
                          _ptr_or0(self.inner.state[p].get("m_scale")),
                          tuple(_ptr_or0(t) for t in (self.inner._inject_noise.get(p) or ())))
                         for p in plist)
            hit = self._mplans.get((gid, pdt, gradless))
            if hit is None or hit[0] != ptrs:
                entries = []
                for p in plist:
                    st = self.inner.state[p]
                    R, C, fac = E.matrixized(p)
                    entries.append(dict(p=p, g=p, R=R, C=C, factored=fac, tensor_id=tids[id(p)], m=st["m"],
                                        m_scale=st.get("m_scale"), block4=st.get("m_block", 0),
                                        noise=self.inner._inject_noise.get(p)))
                group = self.param_groups[gid]
                plan = E.Plan(L.OPT_ADAKAON, L.MOM_CODE[group["momentum_dtype"]], entries, plist[0].device, pdt,
                              pdt)
                idx = torch.tensor([plan.descs[i].ws_scal + 2 for i in range(len(plist))], dtype=torch.int64,
                                   device=plist[0].device)
                hit = (ptrs, plan, [tids[id(p)] for p in plist], idx)
                self._mplans[(gid, pdt, gradless)] = hit
            out.append((gid, pdt, hit[1], hit[2], hit[3]))
        return out

    def _hyper(self, gid: int, pdt: int, step: int | None = None) -> L.KaonHyper:
        h = L.KaonHyper()
        h.p_dtype = h.g_dtype = pdt
        h.codec = L.MOM_CODE[self.param_groups[gid]["momentum_dtype"]]
        h.step = (self.inner._t if step is None else step) & 0xFFFFFFFF
        h.seed = self.inner.sr_seed
        if getattr(self.inner, "reduction_order", "canonical") == "torch":
            h.flags |= L.F_TORCH_ORDER  # the momentum norms' sums in torch CPU's order
        return h

    # ---------------------------------------------------------- perturbation
    @torch.no_grad()
    def _global_mnorm(self, plans: list | None = None) -> float:
        """||m|| over every momentum: per-tensor sums of squares on the GPU, added in
        param order in fp32, fp32 square root (msam.py:191-199)."""
        lib = L.lib()
        tids, vals = [], []
        for gid, pdt, plan, ptids, idx in (self._momentum_plans() if plans is None else plans):
            dev = plan.workspace.device
            L.check(lib.kaon_momentum_sumsq(ctypes.byref(plan.launch), ctypes.byref(self._hyper(gid, pdt)),
                                            E.stream_handle(dev)), "kaon_momentum_sumsq")
            vals.append(plan.workspace.index_select(0, idx))
            tids.append(np.asarray(ptids))
        if not vals:
            return 0.0
        v = np.concatenate([t.cpu().numpy() for t in vals])[np.argsort(np.concatenate(tids), kind="stable")]
        # add.accumulate adds left to right in float32: the sequential fold
        sq = np.add.accumulate(v.astype(np.float32), dtype=np.float32)[-1]
        return float(np.sqrt(sq, dtype=np.float32))

    @torch.no_grad()
    def _apply(self, sign: float, step: int | None = None, plans: list | None = None) -> None:
        """Add the perturbation sign * e to every weight with a momentum (msam.py:202-235).
        The SR noise is keyed on ``step`` (default: the inner step count) and stream 0
        for a removal, 2 for a climb."""
        lib = L.lib()
        sid = 0 if sign < 0 else 2
        for gid, pdt, plan, _tids, _idx in (self._momentum_plans() if plans is None else plans):
            group = self.param_groups[gid]
            if self.norm == "tensor":
                # each tensor's radius from its current momentum (msam.py:219-222); m is
                # unchanged between a climb and its removal, so the round trip is exact
                h = self._hyper(gid, pdt, step)
                dev = plan.workspace.device
                L.check(lib.kaon_momentum_sumsq(ctypes.byref(plan.launch), ctypes.byref(h), E.stream_handle(dev)),
                        "kaon_momentum_sumsq")
                L.check(lib.kaon_msam_apply_tensor(ctypes.byref(plan.launch), ctypes.byref(h), sign * self.rho,
                                                   self.eps, sid, E.stream_handle(dev)), "kaon_msam_apply_tensor")
                continue
            if self.norm == "global":
                factor, bound = sign * self.rho / (self._mnorm + self.eps), math.inf
            else:
                if sign > 0 and gid not in self._eclamp:
                    self._eclamp[gid] = abs(self.rho) * group.get("clip_threshold", 1.0) * group["lr"]
                factor, bound = sign * self.rho, self._eclamp.get(gid, 0.0)
            h = self._hyper(gid, pdt, step)
            L.check(lib.kaon_msam_apply(ctypes.byref(plan.launch), ctypes.byref(h), factor, bound, sid,
                                        E.stream_handle(plan.workspace.device)), "kaon_msam_apply")

    # ---------------------------------------------------------------- step
    @torch.no_grad()
    def step(self, closure: Any = None) -> Any:
        if not self._train_mode:
            raise RuntimeError(
                "MSAM.step() called outside train mode. Call optimizer.train() before the "
                "training step (and optimizer.eval() before sampling / checkpointing).")
        if self.rho != 0.0 and any(p.dtype == torch.float16 for g in self.param_groups for p in g["params"]):
            # the perturbation is an add_stochastic_ write, which the reference has for
            # bf16 and fp32 targets only (_stochastic_rounding.py:55-68)
            raise NotImplementedError(
                "add_stochastic_ for target dtype torch.float16 is not implemented; currently only "
                "torch.bfloat16 and torch.float32 are supported")
        if self._fused and self.norm != "tensor":
            # The removal and the climb are folded into the Adakaon apply of the params
            # that step.  A param with a momentum but no gradient this step is not
            # stepped; MSAM still removes its climb and climbs again along its
            # (unchanged) momentum (msam.py:384-403), in passes of their own keyed on
            # the same step.
            idle = self._momentum_plans(gradless=True) if self.rho != 0.0 else []
            if self._has_e and idle:
                self._apply(-1.0, self.inner._t + 1, plans=idle)
            if self.norm == "global":
                nk = {"remove": self._has_e, "bound_old": {g: math.inf for g in range(len(self.param_groups))},
                      "k": -self.rho / (self._mnorm + self.eps), "climb": False, "eclamp": {}}
            else:  # rho = -k in the fused removal / climb (Nekaon's form)
                nk = {"remove": self._has_e, "bound_old": dict(self._eclamp), "k": -self.rho, "eclamp": {}}
            self._has_e = False
            self._eclamp = {}
            loss = self.inner._step_impl(closure, nk=nk)
            if self.norm == "none":
                if self.rho != 0.0 and self._has_momentum():
                    # bounds frozen at this climb: the stepped groups' from the fused climb,
                    # the others' by _apply below
                    self._eclamp = nk["eclamp"]
                    if idle:
                        self._apply(+1.0, plans=idle)
                    self._has_e = True
                return loss
        else:
            if self._has_e:  # keyed on the coming step, as the fused removal is
                self._apply(-1.0, self.inner._t + 1)
                self._has_e = False
            self._eclamp = {}
            loss = self.inner.step(closure)
            if self.norm in ("none", "tensor"):
                if self.rho != 0.0 and self._has_momentum():
                    self._apply(+1.0)
                    self._has_e = True
                return loss
        if self.rho != 0.0:
            plans = self._momentum_plans()
            self._mnorm = self._global_mnorm(plans)
            if self._mnorm > 0.0:
                self._apply(+1.0, plans=plans)
                self._has_e = True
        return loss

    # ------------------------------------------------------------ eval/train
    @torch.no_grad()
    def eval(self) -> None:  # noqa: A003 - mirrors MSAM.eval()
        if self._train_mode and self._has_e:
            self._apply(-1.0)
        self._train_mode = False

    @torch.no_grad()
    def train(self) -> None:
        if not self._train_mode and self._has_e:
            self._apply(+1.0)
        self._train_mode = True

    # ------------------------------------------------------------ delegation
    def zero_grad(self, set_to_none: bool = True) -> None:  # noqa: FBT001, FBT002
        self.inner.zero_grad(set_to_none=set_to_none)

    def add_param_group(self, param_group: dict[str, Any]) -> None:
        if not hasattr(self, "inner"):
            return super().add_param_group(param_group)
        self.inner.add_param_group(param_group)
        self._mplans.clear()

    def state_dict(self) -> dict[str, Any]:
        sd = self.inner.state_dict()
        sd["msam"] = {}
        return sd

    def load_state_dict(self, state_dict: dict[str, Any]) -> None:
        """msam.py:409-421: checkpoints are saved in eval mode, so no climb is
        active after loading."""
        sd = dict(state_dict)
        sd.pop("msam", None)
        sd.pop("_autolr", None)
        self.inner.load_state_dict(sd)
        self.param_groups = self.inner.param_groups
        self._train_mode = True
        self._has_e = False
        self._mnorm = 0.0
        self._eclamp = {}
        self._mplans.clear()
