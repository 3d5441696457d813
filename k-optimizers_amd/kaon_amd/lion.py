"""Lion on the MI355X HIP step.

Constructor, knobs and state layout follow the reference ``kaon.Lion``
(src/kaon/lion.py:152-241); the update is lion.py:454-485: sign of the
interpolated momentum, momentum EMA through the codec, decoupled WD (``wd``,
not ``lr*wd``), cautious masking, ``*lr``, SR / RN / fp32 write.  One launch
sequence per param group and dtype pair (``kaon_lion_step``).
"""
from __future__ import annotations

import ctypes
from typing import Any, Iterable

import torch

from . import _engine as E
from . import _lib as L
from ._base import (FOREACH_BATCH_CUTOFF, _FOURBIT_BLOCK, KaonOptimizer, init_momentum_state, validate_common,
                    validate_reduction_order)


class Lion(KaonOptimizer):
    _OPT = L.OPT_LION
    _NAME = "Lion"
    _HALF = True

    def __init__(
        self,
        params: Iterable[Any],
        lr: float = 1e-4,
        betas: tuple[float, float] = (0.9, 0.99),
        weight_decay: float = 0.0,
        *,
        momentum_dtype: str = "bfloat16",
        momentum_4bit_block: int = _FOURBIT_BLOCK,
        cautious: bool = True,
        gradient_centralization: bool = True,
        bf16_method: str = "stochastic_rounding",
        foreach: bool = True,
        foreach_batch_cutoff: int = FOREACH_BATCH_CUTOFF,
        foreach_stack_budget: int | None = None,
        auto_lr: bool = False,
        auto_lr_scale: float = 1.0,
        auto_lr_fuse_rel: float = 0.0,
        auto_lr_d0: float | None = None,
        reduction_order: str = "canonical",
    ) -> None:
        beta1, beta2 = validate_common(lr, betas, momentum_dtype, bf16_method, foreach_batch_cutoff, auto_lr)
        self.reduction_order = validate_reduction_order(reduction_order)
        if weight_decay < 0.0:
            raise ValueError(f"weight_decay must be >= 0, got {weight_decay}")
        defaults = {
            "lr": lr,
            "betas": (beta1, beta2),
            "weight_decay": weight_decay,
            "momentum_dtype": momentum_dtype,
            "momentum_4bit_block": momentum_4bit_block,
            "cautious": cautious,
            "gradient_centralization": gradient_centralization,
            "bf16_method": bf16_method,
        }
        super().__init__(params, defaults)
        self._foreach = foreach
        self._foreach_batch_cutoff = foreach_batch_cutoff
        self._foreach_stack_budget = foreach_stack_budget

    @torch.no_grad()
    def _init_state(self, p: torch.Tensor, state: dict[str, Any], group: dict[str, Any]) -> None:
        """lion.py:210-241: the single momentum buffer in the codec layout."""
        init_momentum_state(state, p.grad, group)
        if p.dtype in (torch.bfloat16, torch.float16) and group["bf16_method"] == "kahan":
            state["shift"] = torch.zeros_like(p, memory_format=torch.contiguous_format)

    def _hyper(self, group: dict[str, Any], pdt: int, gdt: int) -> L.KaonHyper:
        beta1, beta2 = group["betas"]
        wd = group["weight_decay"]
        h = L.KaonHyper()
        h.lr = group["lr"]
        h.b1, h.b2 = beta1, beta2
        h.a1, h.a2 = 1.0 - beta1, 1.0 - beta2
        h.wdl = wd
        flags = L.F_MOMENTUM
        if group["gradient_centralization"]:
            flags |= L.F_GC
            if self.centralize_grads_in_place:
                flags |= L.F_GC_WRITE  # the apply stores the centralized gradient
        if group["cautious"]:
            flags |= L.F_CAUTIOUS
        if wd != 0:
            flags |= L.F_WD
        if self.reduction_order == "torch":
            flags |= L.F_TORCH_ORDER
        h.flags = flags
        h.p_dtype, h.g_dtype = pdt, gdt
        h.codec = L.MOM_CODE[group["momentum_dtype"]]
        h.bf16_method = L.BF16_METHOD[group["bf16_method"]]
        h.step = self._t & 0xFFFFFFFF
        h.seed = self.sr_seed
        return h

    @torch.no_grad()
    def _step_impl(self, closure: Any = None, nk: Any = None) -> Any:
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        self._t += 1
        lib = L.lib()
        for gid, group in enumerate(self.param_groups):
            params, pkey = self._stepped(group)
            if not params:
                continue
            for plan, pdt, gdt, dev in self._launches(gid, group, params, pkey):
                hp = self._hyper(group, pdt, gdt)
                L.check(lib.kaon_lion_step(ctypes.byref(plan.launch), ctypes.byref(hp), E.stream_handle(dev)),
                        "kaon_lion_step")
        return loss

    def _build_launches(self, gid: int, group: dict[str, Any], params: list[torch.Tensor],
                        tids: dict[int, int]) -> list:
        codec = L.MOM_CODE[group["momentum_dtype"]]
        out = []
        for (pdt, gdt), plist in self._partitions(params).items():
            plan = self._plan((gid, pdt, gdt), group, plist, codec, tids)
            out.append((plan, pdt, gdt, plist[0].device))
        return out
