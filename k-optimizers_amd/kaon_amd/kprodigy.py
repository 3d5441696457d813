"""KProdigy (parameter-free D adaptation) on the MI355X HIP step.

Constructor, knobs, param-group keys (the D state ``d``, ``d_max``,
``d_numerator``, ``k`` included) and per-param state (``step``, ``s``, ``p0``,
the codec's momentum, ``v`` or ``row`` / ``col``, ``shift``) follow the reference
``kaon.KProdigy`` (src/kaon/kprodigy.py:155-291).  ``step()`` runs, per D scope
(one per group with ``independent_d``, else all groups), the reference's two
passes (``_step_scope``, :306-386):

* pass 1 on the GPU (``kaon_kprodigy_pass1``): the d-scaled momentum EMA, the
  second moment, the ``s`` EMA and each tensor's D statistics;
* the D update on the host, from the per-tensor statistics folded in param
  order in fp32 and the scalar recurrence in double, as the reference does
  after its ``.item()``;
* pass 2 on the GPU (``kaon_kprodigy_pass2``): the update with the new ``d`` and
  the ``dlr`` of the old one.

The ``foreach`` knobs are accepted and have no effect.  A coupled weight decay
(``decouple=False``) folds ``wd * p`` into the gradient of pass 1 (the momentum,
the full or factored second moment and the D statistics, ``_collect_grad``,
:406-414).  fp16 params take fp16 grads and are written by RN or kahan, as the
reference's ``subtract_one_`` writes them.  With gradient centralization on,
pass 2 leaves ``p.grad`` centralized, as the reference's native path does.
``factor_conv_as_matrix=False`` factors the second moment of a weight of 3+
dims over its last two dims (``row`` of shape[:-1], ``col`` of shape[:-2] +
shape[-1:]), each [kh, kw] block on its own, as the reference's per-param path
does (its foreach path cannot unpack those shapes).  SR noise is keyed by
(``sr_seed``, step, param index, element).
"""
from __future__ import annotations

import ctypes
import math
from typing import Any, Iterable

import numpy as np
import torch

from . import _engine as E
from . import _lib as L
from ._base import FOREACH_BATCH_CUTOFF, _FOURBIT_BLOCK, KaonOptimizer, init_momentum_state


class KProdigy(KaonOptimizer):
    _OPT = L.OPT_KPRODIGY
    _NAME = "KProdigy"
    _HALF = True  # fp16 params with fp16 grads: RN / kahan writes (subtract_one_, _backend.py:82-98)

    def __init__(
        self,
        params: Iterable[Any],
        lr: float = 1.0,
        betas: tuple[float, float] = (0.9, 0.999),
        beta3: float | None = None,
        eps: float = 1e-8,
        weight_decay: float = 0.0,
        *,
        decouple: bool = True,
        use_bias_correction: bool = False,
        safeguard_warmup: bool = False,
        d0: float = 1e-6,
        d_coef: float = 1.0,
        growth_rate: float = float("inf"),
        d_update_freq: int = 1,
        slice_p: int = 1,
        independent_d: bool | None = None,
        momentum_dtype: str = "bfloat16",
        momentum_4bit_block: int = _FOURBIT_BLOCK,
        second_moment: str = "full",
        eps_factored: float = 1e-30,
        cautious: bool = False,
        gradient_centralization: bool = True,
        bf16_method: str = "stochastic_rounding",
        factor_conv_as_matrix: bool = True,
        foreach: bool = True,
        foreach_batch_cutoff: int = FOREACH_BATCH_CUTOFF,
        foreach_stack_budget: int | None = None,
    ) -> None:
        # validation in the reference's order and words (kprodigy.py:181-205)
        beta1, beta2 = float(betas[0]), float(betas[1])
        if not d0 > 0.0:
            raise ValueError(f"d0 must be > 0, got {d0}")
        if not lr > 0.0:
            raise ValueError(f"lr must be > 0, got {lr}")
        if not eps > 0.0:
            raise ValueError(f"eps must be > 0, got {eps}")
        if not 0.0 <= beta1 < 1.0:
            raise ValueError(f"betas[0] must be in [0, 1), got {beta1}")
        if not 0.0 <= beta2 < 1.0:
            raise ValueError(f"betas[1] must be in [0, 1), got {beta2}")
        if d_update_freq < 1:
            raise ValueError(f"d_update_freq must be >= 1, got {d_update_freq}")
        if slice_p < 1:
            raise ValueError(f"slice_p must be >= 1, got {slice_p}")
        if momentum_dtype not in ("bfloat16", "float32", "int8", "4bit"):
            raise ValueError(f"momentum_dtype must be bfloat16/float32/int8/4bit, got {momentum_dtype!r}")
        if second_moment not in ("full", "factored"):
            raise ValueError(f"second_moment must be full/factored, got {second_moment!r}")
        if bf16_method not in ("stochastic_rounding", "kahan", "none"):
            raise ValueError(f"bf16_method must be stochastic_rounding/kahan/none, got {bf16_method!r}")
        if foreach_batch_cutoff < 1:
            raise ValueError(f"foreach_batch_cutoff must be >= 1, got {foreach_batch_cutoff}")
        defaults = {
            "lr": lr, "betas": (beta1, beta2), "beta3": beta3, "eps": eps, "weight_decay": weight_decay,
            "decouple": decouple, "use_bias_correction": use_bias_correction, "safeguard_warmup": safeguard_warmup,
            "d": d0, "d0": d0, "d_max": d0, "d_numerator": 0.0, "d_coef": d_coef, "growth_rate": growth_rate,
            "d_update_freq": d_update_freq, "slice_p": slice_p, "k": 0, "momentum_dtype": momentum_dtype,
            "momentum_4bit_block": momentum_4bit_block, "second_moment": second_moment,
            "eps_factored": eps_factored, "cautious": cautious, "gradient_centralization": gradient_centralization,
            "bf16_method": bf16_method, "factor_conv_as_matrix": factor_conv_as_matrix,
        }
        self.d0 = d0
        super().__init__(params, defaults)
        self._independent_d = (len(self.param_groups) > 1) if independent_d is None else independent_d
        self._foreach = foreach
        self._foreach_batch_cutoff = foreach_batch_cutoff
        self._foreach_stack_budget = foreach_stack_budget

    def get_d(self) -> float:
        """Current D estimate (effective learning rate) of the first group."""
        return float(self.param_groups[0].get("d", self.d0))

    @torch.no_grad()
    def _init_state(self, p: torch.Tensor, state: dict[str, Any], group: dict[str, Any]) -> None:
        """kprodigy.py:262-291."""
        factored = group["second_moment"] == "factored" and p.ndim >= 2
        sliced = p.detach().flatten()[:: group["slice_p"]]
        state["step"] = 0
        state["s"] = torch.zeros_like(sliced, dtype=torch.float32, memory_format=torch.contiguous_format)
        if sliced.norm() > 0:
            state["p0"] = sliced.float().clone(memory_format=torch.contiguous_format)
        else:
            state["p0"] = torch.zeros((), device=p.device, dtype=torch.float32)
        if group["betas"][0] > 0:
            init_momentum_state(state, p, group)
        if factored and p.ndim > 2 and not group["factor_conv_as_matrix"]:
            # factored over the last two dims, blocks of [shape[-2], shape[-1]] (kprodigy.py:286-288)
            state["row"] = torch.zeros(p.shape[:-1], dtype=torch.float32, device=p.device)
            state["col"] = torch.zeros(p.shape[:-2] + p.shape[-1:], dtype=torch.float32, device=p.device)
        elif factored:
            R = p.shape[0]
            state["row"] = torch.zeros((R,), dtype=torch.float32, device=p.device)
            state["col"] = torch.zeros((p.numel() // R if R else 0,), dtype=torch.float32, device=p.device)
        else:
            state["v"] = torch.zeros_like(p, dtype=torch.float32, memory_format=torch.contiguous_format)
        if p.dtype in (torch.bfloat16, torch.float16) and group["bf16_method"] == "kahan":
            state["shift"] = torch.zeros_like(p, memory_format=torch.contiguous_format)

    def _entries(self, group: dict[str, Any], params: list[torch.Tensor], tids: dict[int, int]) -> list[dict]:
        out = super()._entries(group, params, tids)
        for e, p in zip(out, params):
            st = self.state[p]
            e.update(pd_s=st["s"], pd_p0=st["p0"], pd_slice=group["slice_p"], full_v="v" in st)
            if "row" in st and st["row"].dim() > 1:  # factored over the last two dims
                e["fb"] = (int(p.shape[-2]), int(p.shape[-1]))
        return out

    def _build_launches(self, gid: int, group: dict[str, Any], params: list[torch.Tensor],
                        tids: dict[int, int]) -> list:
        mom = group["betas"][0] > 0
        codec = L.MOM_CODE[group["momentum_dtype"]] if mom else L.MOM_NONE
        pos = {id(p): i for i, p in enumerate(params)}
        out = []
        for (pdt, gdt), plist in self._partitions(params).items():
            plan = self._plan((gid, pdt, gdt), group, plist, codec, tids)
            # the workspace words holding each tensor's D statistics (num, den)
            words = []
            for i in range(len(plist)):
                words += [plan.descs[i].ws_scal + 2, plan.descs[i].ws_scal + 3]
            stat_idx = torch.tensor(words, dtype=torch.int64, device=plist[0].device)
            out.append((plan, pdt, gdt, plist[0].device, [pos[id(p)] for p in plist], stat_idx))
        return out

    def _hyper(self, group: dict[str, Any], pdt: int, gdt: int, c: dict[str, Any]) -> L.KaonHyper:
        beta1, beta2 = group["betas"]
        wd = group["weight_decay"]
        h = L.KaonHyper()
        h.b1, h.w1 = beta1, 1.0 - beta1
        h.b2, h.w2 = beta2, 1.0 - beta2
        h.eps1 = group["eps_factored"]
        coupled = wd != 0 and not group["decouple"]
        h.wdl = wd if coupled else 0.0
        d, dlr = c["d"], c["dlr"]
        h.pd_tg, h.pd_vval = d * (1.0 - beta1), d * d * (1.0 - beta2)
        h.pd_alpha_s, h.pd_beta3 = c["alpha_s"], c["beta3"]
        h.pd_d = d
        dn = c.get("d_new", d)
        h.pd_dn, h.pd_floor, h.pd_cap = dn, dn * group["eps"], 1.0 / (dn * group["eps"])
        h.pd_dlr, h.pd_wdl = dlr, wd * dlr
        flags = 0
        if group["gradient_centralization"]:
            flags |= L.F_GC
        if group["cautious"]:
            flags |= L.F_CAUTIOUS
        if wd != 0 and group["decouple"]:
            flags |= L.F_WD
        if coupled:
            flags |= L.F_PD_COUPLED
        if group["eps_factored"] > 0:
            flags |= L.F_EPS
        if beta1 > 0:
            flags |= L.F_MOMENTUM
        if group["lr"] > 0.0 and c["should_update_d"]:
            flags |= L.F_PD_STATS
        h.flags = flags
        h.p_dtype, h.g_dtype = pdt, gdt
        h.codec = L.MOM_CODE[group["momentum_dtype"]] if beta1 > 0 else L.MOM_NONE
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
        gids = list(range(len(self.param_groups)))
        scopes = [[g] for g in gids] if self._independent_d else [gids]
        for scope in scopes:
            self._step_scope(scope)
        return loss

    def _step_scope(self, gids: list[int]) -> None:
        """kprodigy.py:306-386."""
        lib = L.lib()
        groups = [self.param_groups[g] for g in gids]
        lead = groups[0]
        beta1, beta2 = lead["betas"]
        beta3 = lead["beta3"] if lead["beta3"] is not None else math.sqrt(beta2)
        k, d, d_max, d0 = lead["k"], lead["d"], lead["d_max"], lead["d0"]
        lr = max(g["lr"] for g in groups)
        bias_correction = (((1 - beta2 ** (k + 1)) ** 0.5) / (1 - beta1 ** (k + 1))
                           if lead["use_bias_correction"] else 1.0)
        dlr = d * lr * bias_correction
        should_update_d = (k % lead["d_update_freq"]) == 0
        d_over_d0 = d / d0
        d_numerator = lead["d_numerator"] * beta3
        c = {"d": d, "dlr": dlr, "beta3": beta3, "should_update_d": should_update_d,
             "alpha_s": (d_over_d0 * d) if lead["safeguard_warmup"] else (d_over_d0 * dlr)}
        # pass 1
        per_group = []
        stats = []  # (group order, param position, device tensor of [num, den] per tensor)
        for order, (gid, group) in enumerate(zip(gids, groups)):
            if group["lr"] not in (lr, 0.0):
                raise RuntimeError("KProdigy: groups sharing one D estimate must use the same lr "
                                   "(or 0 for a frozen group). Use independent_d=True for per-group lr.")
            params, pkey = self._stepped(group)
            launches = self._launches(gid, group, params, pkey) if params else []
            per_group.append((group, params, launches))
            for plan, pdt, gdt, dev, positions, stat_idx in launches:
                hp = self._hyper(group, pdt, gdt, c)
                if plan.any_fb:
                    hp.flags |= L.F_PD_BLOCKFAC
                L.check(lib.kaon_kprodigy_pass1(ctypes.byref(plan.launch), ctypes.byref(hp),
                                                E.stream_handle(dev)), "kaon_kprodigy_pass1")
                if group["lr"] > 0.0 and should_update_d:
                    stats.append((order, positions, plan.workspace.index_select(0, stat_idx)))
        # D update: the per-tensor statistics folded in param order in fp32, then
        # the scalar recurrence in double (kprodigy.py:355-380)
        if should_update_d and lr > 0.0 and stats:
            orders, poss, vals = [], [], []
            for order, positions, t in stats:
                orders.append(np.full(len(positions), order))
                poss.append(np.asarray(positions))
                vals.append(t.cpu().numpy().reshape(-1, 2))
            perm = np.lexsort((np.concatenate(poss), np.concatenate(orders)))
            v = np.concatenate(vals)[perm].astype(np.float32)
            const = np.float32(d_over_d0 * dlr)
            # add.accumulate adds left to right in float32: the sequential fold
            num = np.add.accumulate(const * v[:, 0], dtype=np.float32)[-1]
            den = np.add.accumulate(v[:, 1], dtype=np.float32)[-1]
            if float(den) > 0.0:
                global_num = d_numerator + float(num)
                d_hat = lead["d_coef"] * global_num / float(den)
                if d == d0:
                    d = max(d, d_hat)
                d_max = max(d_max, d_hat)
                d = min(d_max, d * lead["growth_rate"])
                for group in groups:
                    group.update(d_numerator=global_num, d=d, d_max=d_max, d_hat=d_hat)
        c["d_new"] = d
        # pass 2: the new d, the dlr of the old one
        for group, params, launches in per_group:
            for p in params:
                self.state[p]["step"] += 1
            for plan, pdt, gdt, dev, _positions, _idx in launches:
                hp = self._hyper(group, pdt, gdt, c)
                if self.centralize_grads_in_place:
                    hp.flags |= L.F_GC_WRITE  # the apply stores the centralized gradient
                L.check(lib.kaon_kprodigy_pass2(ctypes.byref(plan.launch), ctypes.byref(hp),
                                                E.stream_handle(dev)), "kaon_kprodigy_pass2")
            group["k"] = group["k"] + 1
