"""AdaMuon on the MI355X HIP step.

Constructor, knobs, param-group keys and state layout follow the reference
``kaon.AdaMuon`` (src/kaon/adamuon.py:216-335).  For 2-D and conv params a
step is (adamuon.py:557-593, batched twin :434-501):

1. the momentum of the raw gradient through the codec (``m`` holds it);
2. Newton-Schulz quintic orthogonalization of the (matrixized) momentum, as
   bf16 MFMA GEMMs (zeropower_via_newtonschulz5, :97-118);
3. the factored second moment of the orthogonal factor O, U = O * r * c,
   RMS clip, ``U *= 0.2 * lr``;
4. decoupled weight decay, cautious masking against the gradient, the
   SR / RN / kahan / fp32 write.

1-D params take the Adakaon non-factored path with the update scaled by
``0.2 * lr`` (adamuon.py:594-604), so they step through an Adakaon plan.
``compile`` and the foreach knobs are accepted and have no effect.
"""
from __future__ import annotations

import ctypes
from typing import Any, Iterable

import torch

from . import _engine as E
from . import _lib as L
from ._base import FOREACH_BATCH_CUTOFF, _FOURBIT_BLOCK, KaonOptimizer, init_momentum_state, validate_common

_UPDATE_RMS = 0.2  # adamuon.py:88


class AdaMuon(KaonOptimizer):
    _OPT = L.OPT_ADAMUON
    _NAME = "AdaMuon"
    _HALF = True  # fp16 params with fp16 grads: RN / kahan writes (subtract_one_, _backend.py:82-98)

    def __init__(
        self,
        params: Iterable[Any],
        lr: float = 2e-2,
        betas: tuple[float, float] = (0.95, 0.999),
        eps: tuple[float, float] = (1e-30, 1e-3),
        weight_decay: float = 0.0,
        *,
        ns_steps: int = 2,
        clip_threshold: float = 1.0,
        momentum_dtype: str = "bfloat16",
        momentum_4bit_block: int = _FOURBIT_BLOCK,
        cautious: bool = True,
        gradient_centralization: bool = False,
        bf16_method: str = "stochastic_rounding",
        foreach: bool = True,
        foreach_batch_cutoff: int = FOREACH_BATCH_CUTOFF,
        foreach_stack_budget: int | None = None,
        compile: bool = False,  # noqa: A002 -- the reference's public keyword
        auto_lr: bool = False,
        auto_lr_scale: float = 1.0,
        auto_lr_fuse_rel: float = 0.0,
        auto_lr_d0: float | None = None,
    ) -> None:
        beta1, beta2 = validate_common(lr, betas, momentum_dtype, bf16_method, foreach_batch_cutoff, auto_lr)
        if ns_steps < 1:
            raise ValueError(f"ns_steps must be >= 1, got {ns_steps}")
        if clip_threshold <= 0.0:
            raise ValueError(f"clip_threshold must be > 0, got {clip_threshold}")
        defaults = {
            "lr": lr,
            "betas": (beta1, beta2),
            "eps": (float(eps[0]), float(eps[1])),
            "weight_decay": weight_decay,
            "ns_steps": ns_steps,
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

    @torch.no_grad()
    def _init_state(self, p: torch.Tensor, state: dict[str, Any], group: dict[str, Any]) -> None:
        """adamuon.py:318-335: row/col of the matrixized shape for ndim >= 2, v
        for 1-D; the codec's buffer of the raw grad's momentum; kahan shift."""
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

    def _hyper(self, group: dict[str, Any], pdt: int, gdt: int) -> L.KaonHyper:
        beta1, beta2 = group["betas"]
        eps1 = group["eps"][0]
        lr, wd, clip = group["lr"], group["weight_decay"], group["clip_threshold"]
        h = L.KaonHyper()
        h.lr = _UPDATE_RMS * lr          # update.mul_(_UPDATE_RMS * lr), adamuon.py:588, 603
        h.w1 = 1.0 - beta1
        h.w2 = 1.0 - beta2
        h.eps1 = eps1
        h.wdl = lr * wd                  # delta.add_(p, alpha=lr * wd), adamuon.py:606-608
        h.clip = clip
        flags = 0
        if group["gradient_centralization"]:
            flags |= L.F_GC
        if group["cautious"]:
            flags |= L.F_CAUTIOUS
        if wd != 0:
            flags |= L.F_WD
        if eps1 > 0:
            flags |= L.F_EPS
        mom = beta1 > 0
        if mom:
            flags |= L.F_MOMENTUM
        h.flags = flags
        h.p_dtype, h.g_dtype = pdt, gdt
        h.codec = L.MOM_CODE[group["momentum_dtype"]] if mom else L.MOM_NONE
        h.bf16_method = L.BF16_METHOD[group["bf16_method"]]
        h.ns_steps = int(group["ns_steps"])
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
            for fn, plan, pdt, gdt, dev in self._launches(gid, group, params, pkey):
                hp = self._hyper(group, pdt, gdt)
                L.check(getattr(lib, fn)(ctypes.byref(plan.launch), ctypes.byref(hp), E.stream_handle(dev)), fn)
                self._gc_writeback(group, plan, hp, dev)
        return loss

    def _build_launches(self, gid: int, group: dict[str, Any], params: list[torch.Tensor],
                        tids: dict[int, int]) -> list:
        """The matrices through an AdaMuon plan, the 1-D params through an Adakaon plan
        (hp.lr is already 0.2 * lr, adamuon.py:88, 588)."""
        mom = group["betas"][0] > 0
        codec = L.MOM_CODE[group["momentum_dtype"]] if mom else L.MOM_NONE
        out = []
        for (pdt, gdt), plist in self._partitions(params).items():
            dev = plist[0].device
            mats = [p for p in plist if p.ndim >= 2]
            vecs = [p for p in plist if p.ndim < 2]
            if mats:
                plan = self._plan((gid, pdt, gdt, 2), group, mats, codec, tids, L.OPT_ADAMUON)
                out.append(("kaon_adamuon_step", plan, pdt, gdt, dev))
            if vecs:
                plan = self._plan((gid, pdt, gdt, 1), group, vecs, codec, tids, L.OPT_ADAKAON)
                out.append(("kaon_adakaon_step", plan, pdt, gdt, dev))
        return out
