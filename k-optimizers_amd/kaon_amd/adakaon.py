"""Adakaon on the MI355X HIP step.

Constructor, knobs, param-group keys and state layout follow the reference
``kaon.Adakaon`` (src/kaon/adakaon.py:195-335).  ``step()`` runs the whole
update (GC, factored second moment, RMS clip, momentum codec, decoupled WD,
cautious masking, SR / RN / kahan / fp32 write) as one multi-tensor launch
sequence per param group and dtype pair (``kaon_adakaon_step``).  The
reference's ``foreach`` / ``fused`` / stacking knobs are accepted; the weights
and state come out of one path whatever they say (``fused`` decides only what
``p.grad`` holds afterwards, below).

``p.grad`` after the step follows the reference's path: with GC on, the
default (``fused=False``, the reference's native path, which centralizes
``p.grad`` in place, src/kaon/_backend.py:147-177) stores the centralized
gradient over ``p.grad`` from the apply kernel (``KAON_F_GC_WRITE``);
``fused=True`` does so only for the params the reference's fused step routes
to its native path (``fused_routes_native``) and leaves the others' ``p.grad``
as given, as its fused kernels do (adakaon.py:387-409).

Difference from the reference, by design:
* stochastic rounding draws Philox4x32-10 noise keyed by (``sr_seed``, step,
  param index, element) instead of ``torch.randint`` from the global RNG.
"""
from __future__ import annotations

import ctypes
from typing import Any, Iterable

import torch

from . import _engine as E
from . import _lib as L
from ._base import (FOREACH_BATCH_CUTOFF, _FOURBIT_BLOCK, KaonOptimizer, init_momentum_state, validate_common,
                    validate_reduction_order)


# The reference's one-block tile cap (src/kaon/_fused_triton.py:70): 2^17 padded elements.
_TILE_CAP = 1 << 17


def _next_pow2(n: int) -> int:
    return 1 << max(int(n) - 1, 0).bit_length()


def fused_routes_native(p: torch.Tensor, group: dict[str, Any], tile_cap: int = _TILE_CAP) -> bool:
    """Whether the reference's ``fused=True`` Adakaon sends a param of 2 or more dims
    to its native path, which centralizes ``p.grad`` in place (``_fused_partition``,
    src/kaon/adakaon.py:437-468, with ``fused_eligible`` / ``eff_2d``,
    src/kaon/_fused_triton.py:100-139): momentum off, a bf16 param without
    stochastic rounding, a conv (ndim > 2) with int8 / 4-bit momentum, a dtype
    other than fp32 / bf16, or a one-block tile with 4-bit momentum and an odd
    row length.  The one-block and big-tensor kernels centralize in their own
    registers and leave ``p.grad`` as given.  1-D params are never centralized."""
    if p.ndim < 2 or p.numel() == 0:
        return False
    md = group["momentum_dtype"]
    momentum = group["betas"][0] > 0
    bf_ok = p.dtype != torch.bfloat16 or group["bf16_method"] == "stochastic_rounding"
    conv_ok = p.ndim <= 2 or (p.grad is not None and p.grad.is_contiguous() and md in ("bfloat16", "float32"))
    two_d = momentum and bf_ok and conv_ok and p.is_contiguous() and p.dtype in (torch.float32, torch.bfloat16)
    R = p.shape[0]
    C = p.numel() // R
    tile = _next_pow2(R) * _next_pow2(C)
    one_block = two_d and tile <= tile_cap and not (md == "4bit" and C % 2 != 0)
    big = two_d and tile > tile_cap
    return not (one_block or big)


class Adakaon(KaonOptimizer):
    _OPT = L.OPT_ADAKAON
    _NAME = "Adakaon"
    _HALF = True

    def __init__(
        self,
        params: Iterable[Any],
        lr: float = 1e-3,
        betas: tuple[float, float] = (0.9, 0.999),
        eps: tuple[float, float] = (1e-30, 1e-3),
        weight_decay: float = 0.0,
        *,
        clip_threshold: float = 1.0,
        momentum_dtype: str = "bfloat16",
        momentum_4bit_block: int = _FOURBIT_BLOCK,
        cautious: bool = True,
        gradient_centralization: bool = True,
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
        reduction_order: str = "canonical",
    ) -> None:
        beta1, beta2 = validate_common(lr, betas, momentum_dtype, bf16_method, foreach_batch_cutoff, auto_lr)
        self.reduction_order = validate_reduction_order(reduction_order)
        if clip_threshold <= 0.0:
            raise ValueError(f"clip_threshold must be > 0, got {clip_threshold}")
        defaults = {
            "lr": lr,
            "betas": (beta1, beta2),
            "eps": (float(eps[0]), float(eps[1])),
            "weight_decay": weight_decay,
            "clip_threshold": clip_threshold,
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
        self._fused = bool(fused)
        self._fused_tile_cap = _TILE_CAP if fused_tile_cap is None else int(fused_tile_cap)

    @torch.no_grad()
    def _init_state(self, p: torch.Tensor, state: dict[str, Any], group: dict[str, Any]) -> None:
        """adakaon.py:318-335: row/col for ndim >= 2 (conv matrixized), v for 1-D,
        the codec's momentum buffer when beta1 > 0, kahan shift for bf16 params."""
        grad = p.grad
        if p.ndim >= 2:
            R = grad.shape[0]
            state["row"] = torch.zeros((R,), dtype=torch.float32, device=p.device)
            state["col"] = torch.zeros((grad.numel() // R if R else 0,), dtype=torch.float32, device=p.device)
        else:
            state["v"] = torch.zeros_like(grad, dtype=torch.float32, memory_format=torch.contiguous_format)
        if group["betas"][0] > 0:
            init_momentum_state(state, grad, group)
        if p.dtype in (torch.bfloat16, torch.float16) and group["bf16_method"] == "kahan":
            state["shift"] = torch.zeros_like(p, memory_format=torch.contiguous_format)

    def _entries(self, group: dict[str, Any], params: list[torch.Tensor], tids: dict[int, int]) -> list[dict]:
        out = super()._entries(group, params, tids)
        if self._fused:
            for e, p in zip(out, params):
                e["gc_write"] = fused_routes_native(p, group, self._fused_tile_cap)
        return out

    def _hyper(self, group: dict[str, Any], pdt: int, gdt: int, nk: dict | None, gid: int) -> L.KaonHyper:
        beta1, beta2 = group["betas"]
        eps1 = group["eps"][0]
        lr, wd, clip = group["lr"], group["weight_decay"], group["clip_threshold"]
        h = L.KaonHyper()
        h.lr = lr
        h.w1 = 1.0 - beta1
        h.w2 = 1.0 - beta2
        h.eps1 = eps1
        h.wdl = lr * wd
        h.clip = clip
        flags = 0
        if group["gradient_centralization"]:
            flags |= L.F_GC
            if self.centralize_grads_in_place:
                flags |= L.F_GC_WRITE  # the apply stores the centralized gradient
        if group["cautious"]:
            flags |= L.F_CAUTIOUS
        if wd != 0:
            flags |= L.F_WD
        if eps1 > 0:
            flags |= L.F_EPS
        mom = beta1 > 0
        if mom:
            flags |= L.F_MOMENTUM
        if self.reduction_order == "torch":
            flags |= L.F_TORCH_ORDER
        if nk is not None and mom:
            if nk["remove"] and gid in nk["bound_old"]:
                flags |= L.F_NK_REMOVE
                h.nk_bound_old = nk["bound_old"][gid]
            if nk["k"] != 0.0 and nk.get("climb", True):
                flags |= L.F_NK_CLIMB
                bound = abs(nk["k"]) * group.get("clip_threshold", 1.0) * lr
                h.nk_bound_new = bound
                nk["eclamp"][gid] = bound
            h.nk_k = nk["k"]
        h.flags = flags
        h.p_dtype, h.g_dtype = pdt, gdt
        h.codec = L.MOM_CODE[group["momentum_dtype"]] if mom else L.MOM_NONE
        h.bf16_method = L.BF16_METHOD[group["bf16_method"]]
        h.step = self._t & 0xFFFFFFFF
        h.seed = self.sr_seed
        return h

    @torch.no_grad()
    def _step_impl(self, closure: Any = None, nk: dict | None = None) -> Any:
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
                hp = self._hyper(group, pdt, gdt, nk, gid)
                if not plan.any_gc_write:
                    hp.flags &= ~L.F_GC_WRITE
                L.check(lib.kaon_adakaon_step(ctypes.byref(plan.launch), ctypes.byref(hp), E.stream_handle(dev)),
                        "kaon_adakaon_step")
        return loss

    def _build_launches(self, gid: int, group: dict[str, Any], params: list[torch.Tensor],
                        tids: dict[int, int]) -> list:
        mom = group["betas"][0] > 0
        codec = L.MOM_CODE[group["momentum_dtype"]] if mom else L.MOM_NONE
        out = []
        for (pdt, gdt), plist in self._partitions(params).items():
            plan = self._plan((gid, pdt, gdt), group, plist, codec, tids)
            out.append((plan, pdt, gdt, plist[0].device))
        return out
