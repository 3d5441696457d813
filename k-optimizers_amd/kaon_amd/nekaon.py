"""Nekaon on the MI355X HIP step: Momentum-SAM (``norm="none"``, ``rho = -k``)
over Adakaon, with the lookahead fused into the Adakaon apply pass.

Reference: src/kaon/nekaon.py:122-185 (preset, low-VRAM split),
src/kaon/msam.py:169-235 (frozen per-element climb bound, perturbation),
:294-311 (eval/train), :375-406 (step), :409-421 (load).  The reference
touches the weights three times per step (remove the previous climb, inner
step, climb along the new momentum); here the removal, the update and the new
climb are three stochastic roundings of one register value, written once
(SR noise streams 0, 1 and 2).
"""
from __future__ import annotations

import ctypes
from collections import defaultdict
from typing import Any, Iterable

import torch

from . import _engine as E
from . import _lib as L
from .adakaon import Adakaon


class Nekaon(torch.optim.Optimizer):
    def __init__(
        self,
        params: Iterable[Any],
        lr: float = 1e-3,
        k: float = 1.5,
        betas: tuple[float, float] = (0.5, 0.999),
        weight_decay: float = 0.1,
        momentum_dtype: str = "4bit",
        *,
        low_vram_above: int | None = None,
        low_vram_lr_ratio: float = 0.5,
        auto_lr: bool = False,
        auto_lr_scale: float = 1.0,
        auto_lr_fuse_rel: float = 0.0,
        auto_lr_d0: float | None = None,
        **adakaon_kwargs: Any,
    ) -> None:
        if k < 0.0:
            raise ValueError(f"k must be >= 0 (lookahead steps), got {k}")
        if betas[0] <= 0.0:
            raise ValueError("Nekaon requires betas[0] > 0 (the lookahead rides the momentum)")
        if auto_lr:
            raise NotImplementedError("kaon_amd: auto_lr (the DoWG LR controller) is not part of this build")
        if low_vram_above is not None:
            if low_vram_above < 0:
                raise ValueError(f"low_vram_above must be >= 0, got {low_vram_above}")
            params = list(params)
            if params and isinstance(params[0], dict):
                raise TypeError(
                    "low_vram_above does not support param-group dicts — pass a flat "
                    "parameter iterable; Nekaon builds its own small/big groups by tensor size.")
            small = [p for p in params if p.numel() <= low_vram_above]
            big = [p for p in params if p.numel() > low_vram_above]
            if not small and not big:
                raise ValueError("Nekaon got no parameters")
            groups: list[dict[str, Any]] = []
            if small:
                groups.append({"params": small})
            if big:
                groups.append({"params": big, "lr": lr * low_vram_lr_ratio, "betas": (0.0, betas[1])})
            params = groups
        inner = Adakaon(params, lr=lr, betas=betas, weight_decay=weight_decay,
                        momentum_dtype=momentum_dtype, **adakaon_kwargs)
        # torch.optim.Optimizer bookkeeping (hooks, LR-scheduler compatibility);
        # the param groups and defaults are the inner optimizer's
        super().__init__([p for g in inner.param_groups for p in g["params"]], dict(inner.defaults))
        self.inner = inner
        self.base_optimizer = inner
        self.param_groups = self.inner.param_groups
        self.defaults = self.inner.defaults
        self.state = defaultdict(dict)   # MSAM keeps no per-param state of its own
        self.k = float(k)
        self.rho = -float(k)
        self.norm = "none"
        self.eps = 1e-12
        self._train_mode = True
        self._has_e = False
        self._eclamp: dict[int, float] = {}   # per-group climb bound, frozen at climb time

    # ---------------------------------------------------------------- step
    @torch.no_grad()
    def step(self, closure: Any = None) -> Any:
        if not self._train_mode:
            raise RuntimeError(
                "MSAM.step() called outside train mode. Call optimizer.train() before the "
                "training step (and optimizer.eval() before sampling / checkpointing).")
        nk = {"remove": self._has_e, "bound_old": dict(self._eclamp), "k": self.k, "eclamp": {}}
        self._has_e = False
        self._eclamp = {}
        loss = self.inner._step_impl(closure, nk=nk)
        if self.rho != 0.0 and self._momentum_params():
            self._eclamp = nk["eclamp"]
            self._has_e = True
        return loss

    def _momentum_params(self) -> list[tuple[torch.Tensor, dict[str, Any], dict[str, Any], int]]:
        out = []
        for gid, group in enumerate(self.param_groups):
            for p in group["params"]:
                st = self.inner.state.get(p)
                if st and "m" in st:
                    out.append((p, st, group, gid))
        return out

    # ------------------------------------------------------------ eval/train
    @torch.no_grad()
    def _apply(self, sign: float) -> None:
        """p += clamp(nan_to_num(sign*rho*m), +-bound) with the frozen bound (msam.py:202-235)."""
        factor = sign * self.rho
        sid = 0 if sign < 0 else 2
        by_group: dict[tuple[int, int], list[torch.Tensor]] = {}
        for p, _st, group, gid in self._momentum_params():
            by_group.setdefault((gid, E.dtype_code(p.dtype)), []).append(p)
        tids = self.inner._tensor_ids()
        for (gid, pdt), plist in by_group.items():
            group = self.param_groups[gid]
            if sign > 0 and gid not in self._eclamp:
                self._eclamp[gid] = abs(self.rho) * group.get("clip_threshold", 1.0) * group["lr"]
            bound = self._eclamp.get(gid, 0.0)
            entries = []
            for p in plist:
                st = self.inner.state[p]
                R, C, fac = E.matrixized(p)
                entries.append(dict(p=p, g=p, R=R, C=C, factored=fac, tensor_id=tids[id(p)], m=st["m"],
                                    m_scale=st.get("m_scale"), block4=st.get("m_block", 0),
                                    noise=self.inner._inject_noise.get(p)))
            codec = L.MOM_CODE[group["momentum_dtype"]]
            plan = E.Plan(L.OPT_ADAKAON, codec, entries, plist[0].device)
            h = L.KaonHyper()
            h.p_dtype = pdt
            h.g_dtype = pdt
            h.codec = codec
            h.step = self.inner._t & 0xFFFFFFFF
            h.seed = self.inner.sr_seed
            L.check(L.lib().kaon_msam_apply(ctypes.byref(plan.launch), ctypes.byref(h), factor, bound, sid,
                                            E.stream_handle(plist[0].device)), "kaon_msam_apply")
            # the plan's tables must outlive the launch
            torch.cuda.current_stream(plist[0].device).synchronize()

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

    def state_dict(self) -> dict[str, Any]:
        sd = self.inner.state_dict()
        sd["msam"] = {}
        return sd

    def load_state_dict(self, state_dict: dict[str, Any]) -> None:
        """MSAM.load_state_dict (msam.py:409-421): restore the inner optimizer;
        MSAM keeps no persistent state, checkpoints are saved in eval mode
        (unperturbed weights), so no climb is active after loading."""
        sd = dict(state_dict)
        sd.pop("msam", None)
        sd.pop("_autolr", None)
        self.inner.load_state_dict(sd)
        self.param_groups = self.inner.param_groups
        self._train_mode = True
        self._has_e = False
        self._eclamp = {}
        self._has_e = False
        self._eclamp = {}
