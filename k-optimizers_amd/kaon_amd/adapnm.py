"""AdaPNM on the MI355X HIP step.

Constructor, knobs, param-group keys (the per-group ``step`` included) and
state layout follow the reference ``kaon.AdaPNM`` (src/kaon/adapnm.py:344-500):
two momentum buffers ``m_pos`` / ``m_neg`` through the shared codec layout,
whose roles alternate with the step parity (:588-596); a factored second
moment (``row`` / ``col``) for ndim >= 2 with conv kernels matrixized, a full
``v`` (and ``max_v`` under ``ams_bound``) for 1-D params.  ``step()`` runs the
whole update (decoupled WD, second moment with bias correction, EMA of the
positive buffer with the raw gradient at decay beta1^2, positive-negative mix,
RMS clip, lr / (1 - beta1^t), cautious masking, SR / RN / kahan / fp32 write)
as one launch sequence per param group and dtype pair (``kaon_adapnm_step``).
The ``foreach`` / ``fused`` / stacking knobs are accepted and have no effect.

Differences from the reference, by design: gradients are read, never written
(GC happens in registers); stochastic rounding draws Philox4x32-10 noise keyed
by (``sr_seed``, group step, param index, element) instead of ``torch.randint``.
"""
from __future__ import annotations

import ctypes
import math
from typing import Any, Iterable

import torch

from . import _engine as E
from . import _lib as L
from ._base import FOREACH_BATCH_CUTOFF, _FOURBIT_BLOCK, KaonOptimizer, init_momentum_state


class AdaPNM(KaonOptimizer):
    _OPT = L.OPT_ADAPNM
    _NAME = "AdaPNM"
    _HALF = True  # fp16 params with fp16 grads: RN / kahan writes (subtract_one_, _backend.py:82-98)

    def __init__(
        self,
        params: Iterable[Any],
        lr: float = 1e-3,
        betas: tuple[float, float] = (0.8, 0.999),
        beta0: float = 0.5,
        eps: float = 1e-8,
        weight_decay: float = 0.0,
        *,
        clip_threshold: float = 1.0,
        cautious: bool = True,
        gradient_centralization: bool = True,
        ams_bound: bool = False,
        momentum_dtype: str = "bfloat16",
        momentum_4bit_block: int = _FOURBIT_BLOCK,
        bf16_method: str = "stochastic_rounding",
        foreach: bool = True,
        foreach_batch_cutoff: int = FOREACH_BATCH_CUTOFF,
        foreach_stack_budget: int | None = None,
        fused: bool = False,
        fused_tile_cap: int | None = None,
        auto_lr: bool = False,
        auto_lr_scale: float = 1.0,
        auto_lr_fuse_rel: float = 0.0,
        auto_lr_d0: float | None = None,
    ) -> None:
        # validation in the reference's order and words (adapnm.py:371-398)
        beta1, beta2 = float(betas[0]), float(betas[1])
        if not 0.0 <= beta1 < 1.0:
            raise ValueError(f"betas[0] must be in [0, 1), got {beta1}")
        if not 0.0 <= beta2 < 1.0:
            raise ValueError(f"betas[1] must be in [0, 1), got {beta2}")
        if not 0.0 <= beta0 <= 1.0:
            raise ValueError(f"beta0 must be in [0, 1], got {beta0}")
        if lr < 0.0:
            raise ValueError(f"lr must be >= 0, got {lr}")
        if eps < 0.0:
            raise ValueError(f"eps must be >= 0, got {eps}")
        if clip_threshold < 0.0:
            raise ValueError(f"clip_threshold must be >= 0, got {clip_threshold}")
        if weight_decay < 0.0:
            raise ValueError(f"weight_decay must be >= 0, got {weight_decay}")
        if momentum_dtype not in ("bfloat16", "float32", "int8", "4bit"):
            raise ValueError(f"momentum_dtype must be bfloat16/float32/int8/4bit, got {momentum_dtype!r}")
        if bf16_method not in ("stochastic_rounding", "kahan", "none"):
            raise ValueError(f"bf16_method must be stochastic_rounding/kahan/none, got {bf16_method!r}")
        if foreach_batch_cutoff < 1:
            raise ValueError(f"foreach_batch_cutoff must be >= 1, got {foreach_batch_cutoff}")
        if auto_lr:
            raise NotImplementedError("kaon_amd: auto_lr (the DoWG LR controller) is not part of this build")
        defaults = {
            "lr": lr,
            "betas": (beta1, beta2),
            "beta0": float(beta0),
            "eps": float(eps),
            "clip_threshold": float(clip_threshold),
            "weight_decay": weight_decay,
            "cautious": cautious,
            "gradient_centralization": gradient_centralization,
            "ams_bound": ams_bound,
            "momentum_dtype": momentum_dtype,
            "momentum_4bit_block": momentum_4bit_block,
            "bf16_method": bf16_method,
            "step": 0,
        }
        super().__init__(params, defaults)
        self._foreach = foreach
        self._foreach_batch_cutoff = foreach_batch_cutoff
        self._foreach_stack_budget = foreach_stack_budget
        self._fused = bool(fused)
        # as Adakaon: native centralize_grads_ (adapnm.py:614-615); the fused kernels
        # centralize in-kernel (adapnm.py:660-665 only for the native subset)
        self.centralize_grads_in_place = not self._fused

    @torch.no_grad()
    def _init_state(self, p: torch.Tensor, state: dict[str, Any], group: dict[str, Any]) -> None:
        """adapnm.py:482-500: row/col for ndim >= 2 (conv matrixized), v (and max_v
        under ams_bound) for 1-D, the two momenta, kahan shift for bf16 params."""
        grad = p.grad
        if p.ndim >= 2:
            R = grad.shape[0]
            state["row"] = torch.zeros((R,), dtype=torch.float32, device=p.device)
            state["col"] = torch.zeros((grad.numel() // R if R else 0,), dtype=torch.float32, device=p.device)
        else:
            state["v"] = torch.zeros_like(grad, dtype=torch.float32, memory_format=torch.contiguous_format)
            if group["ams_bound"]:
                state["max_v"] = torch.zeros_like(grad, dtype=torch.float32, memory_format=torch.contiguous_format)
        init_momentum_state(state, grad, group, "m_pos")
        init_momentum_state(state, grad, group, "m_neg")
        if p.dtype in (torch.bfloat16, torch.float16) and group["bf16_method"] == "kahan":
            state["shift"] = torch.zeros_like(p, memory_format=torch.contiguous_format)

    def _entries(self, group: dict[str, Any], params: list[torch.Tensor], tids: dict[int, int]) -> list[dict]:
        out = super()._entries(group, params, tids)
        for e, p in zip(out, params):
            st = self.state[p]
            e.update(m=st["m_pos"], m_scale=st.get("m_pos_scale"), m2=st["m_neg"], m2_scale=st.get("m_neg_scale"),
                     max_v=st.get("max_v"), block4=st.get("m_pos_block", 0))
        return out

    @staticmethod
    def _coeffs(group: dict[str, Any]) -> dict[str, float]:
        """The per-step scalars in double precision (adapnm.py:998-1016)."""
        beta1, beta2 = group["betas"]
        beta0 = group["beta0"]
        step = group["step"]
        bc1 = 1.0 - beta1 ** step
        return {
            "beta1_sq": beta1 * beta1,
            "noise_norm": math.sqrt((1.0 + beta0) ** 2 + beta0 ** 2),
            "bc2_sq": math.sqrt(1.0 - beta2 ** step),
            "step_size": group["lr"] / bc1,
        }

    def _hyper(self, group: dict[str, Any], pdt: int, gdt: int) -> L.KaonHyper:
        beta1, beta2 = group["betas"]
        beta0, eps = group["beta0"], group["eps"]
        lr, wd = group["lr"], group["weight_decay"]
        c = self._coeffs(group)
        h = L.KaonHyper()
        h.lr = c["step_size"]
        h.b1, h.a1 = c["beta1_sq"], 1.0 - c["beta1_sq"]
        h.b2, h.a2 = beta2, 1.0 - beta2
        h.w2 = 1.0 - beta2
        h.eps1 = eps
        h.wdl = 1.0 - lr * wd
        h.clip = group["clip_threshold"]
        h.pn_pos, h.pn_neg, h.pn_rnorm = 1.0 + beta0, -beta0, 1.0 / c["noise_norm"]
        h.bc2 = c["bc2_sq"]
        flags = L.F_MOMENTUM
        if group["gradient_centralization"]:
            flags |= L.F_GC
        if group["cautious"]:
            flags |= L.F_CAUTIOUS
        if wd != 0:
            flags |= L.F_WD
        if eps > 0:
            flags |= L.F_EPS
        if group["ams_bound"]:
            flags |= L.F_AMS
        h.flags = flags
        h.p_dtype, h.g_dtype = pdt, gdt
        h.codec = L.MOM_CODE[group["momentum_dtype"]]
        h.bf16_method = L.BF16_METHOD[group["bf16_method"]]
        h.step = group["step"] & 0xFFFFFFFF
        h.seed = self.sr_seed
        return h

    @torch.no_grad()
    def _step_impl(self, closure: Any = None, nk: Any = None) -> Any:
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        lib = L.lib()
        for gid, group in enumerate(self.param_groups):
            params, pkey = self._stepped(group)
            launches = self._launches(gid, group, params, pkey) if params else []
            group["step"] += 1
            for plan, pdt, gdt, dev in launches:
                hp = self._hyper(group, pdt, gdt)
                L.check(lib.kaon_adapnm_step(ctypes.byref(plan.launch), ctypes.byref(hp), E.stream_handle(dev)),
                        "kaon_adapnm_step")
                self._gc_writeback(group, plan, hp, dev)
        return loss

    def _build_launches(self, gid: int, group: dict[str, Any], params: list[torch.Tensor],
                        tids: dict[int, int]) -> list:
        codec = L.MOM_CODE[group["momentum_dtype"]]
        out = []
        for (pdt, gdt), plist in self._partitions(params).items():
            plan = self._plan((gid, pdt, gdt), group, plist, codec, tids)
            out.append((plan, pdt, gdt, plist[0].device))
        return out
