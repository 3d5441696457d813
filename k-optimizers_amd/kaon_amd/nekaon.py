"""Nekaon on the MI355X HIP step: the Momentum-SAM preset ``norm="none"``,
``rho = -k`` over Adakaon (src/kaon/nekaon.py:85-185: preset, low-VRAM split),
with the lookahead fused into the Adakaon apply pass.

The reference touches the weights three times per step (remove the previous
climb, inner step, climb along the new momentum, src/kaon/msam.py:375-406);
here the removal, the update and the new climb are three stochastic roundings
of one register value, written once (SR noise streams 0, 1 and 2).  Step,
eval/train, the frozen climb bound and loading are :class:`MSAM`'s.
"""
from __future__ import annotations

from typing import Any, Iterable

from .adakaon import Adakaon
from .msam import MSAM


class Nekaon(MSAM):
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
        inner = Adakaon(params, lr=lr, betas=betas, weight_decay=weight_decay, momentum_dtype=momentum_dtype,
                        **adakaon_kwargs)
        self._bind(inner, rho=-float(k), norm="none", eps=1e-12)
        self.k = float(k)
