"""Shared optimizer plumbing: state layout, plan cache, checkpoint I/O.

State keys, dtypes and shapes are the reference's (K-Optimizers "kaon"
0.7.4), so checkpoints move between the two libraries:
  Adakaon  src/kaon/adakaon.py:318-335    Lion  src/kaon/lion.py:210-241
  codecs   src/kaon/_momentum_codec.py:253-406 (init_state of each codec)
  loading  src/kaon/_momentum_codec.py:417-452 (dtype-preserving load)
"""
from __future__ import annotations

import ctypes
from itertools import chain
from typing import Any, Iterable

import torch
import torch.optim.optimizer as _topt

from . import _engine as E
from . import _keys as K
from . import _lib as L

_FOURBIT_BLOCK = 128          # src/kaon/_momentum_codec.py:59
FOREACH_BATCH_CUTOFF = 2_000_000  # src/kaon/_backend.py:53 (accepted for API compatibility)


def fourbit_block_size(numel: int, block: int) -> int:
    """4-bit absmax block for a tensor of ``numel`` elements (_momentum_codec.py:192-200)."""
    return numel if block <= 0 else (min(block, numel) if numel > 0 else 1)


def init_momentum_state(state: dict[str, Any], grad: torch.Tensor, group: dict[str, Any], prefix: str = "m") -> None:
    """Allocate a momentum buffer exactly as the reference codecs do, under the keys
    ``prefix``, ``prefix_scale``, ``prefix_numel``, ``prefix_block`` (AdaPNM's two
    buffers use "m_pos" and "m_neg", src/kaon/adapnm.py:451-479)."""
    md = group["momentum_dtype"]
    if md in ("bfloat16", "float32"):
        state[prefix] = torch.zeros_like(grad, dtype=torch.bfloat16 if md == "bfloat16" else torch.float32,
                                         memory_format=torch.contiguous_format)
    elif md == "int8":
        state[prefix] = torch.zeros_like(grad, dtype=torch.int8, memory_format=torch.contiguous_format)
        state[f"{prefix}_scale"] = torch.ones((grad.shape[0],) + (1,) * (grad.ndim - 1) if grad.ndim >= 2 else (),
                                              dtype=torch.float32, device=grad.device)
    else:
        numel = grad.numel()
        bs = fourbit_block_size(numel, group["momentum_4bit_block"])
        nblocks = (numel + bs - 1) // bs
        state[prefix] = torch.full(((numel + 1) // 2,), 0x88, dtype=torch.uint8, device=grad.device)
        state[f"{prefix}_scale"] = torch.ones(nblocks, dtype=torch.float32, device=grad.device)
        state[f"{prefix}_numel"] = numel
        state[f"{prefix}_block"] = bs


def load_state_dict_preserving_dtypes(optimizer: torch.optim.Optimizer, state_dict: dict[str, Any]) -> None:
    """torch's load_state_dict with every state tensor kept as saved
    (_momentum_codec.py:417-452).

    torch casts each state tensor to the param's dtype on load.  The reference
    casts it back afterwards, which is exact for fp32 params; with bf16 params
    the fp32 row/col/v/scale state would come back rounded to bf16.  Here a
    tensor whose dtype torch changed is replaced by the saved tensor itself,
    moved to the param's device, so a resume is byte-identical for any param
    dtype.  Keys and layout are the reference's, so checkpoints move both ways.
    """
    saved = state_dict.get("state", {})
    torch.optim.Optimizer.load_state_dict(optimizer, state_dict)
    params = [p for group in optimizer.param_groups for p in group["params"]]
    for i, p in enumerate(params):
        s = saved.get(i)
        if s is None or p not in optimizer.state:
            continue
        st = optimizer.state[p]
        for key, v in s.items():
            t = st.get(key)
            if torch.is_tensor(v) and torch.is_tensor(t) and t.dtype != v.dtype:
                st[key] = v.detach().to(device=p.device, copy=True)


REDUCTION_ORDERS = ("canonical", "torch")


def validate_reduction_order(order: str) -> str:
    """``reduction_order`` (no counterpart in the reference): "canonical" sums the step's
    fp32 reductions in the library's fixed 64-lane order (the default; the faster form);
    "torch" sums them in torch CPU's order (KAON_F_TORCH_ORDER), which reproduces the
    reference's results bit for bit and costs the clip norm's n/8 sequential fma chains."""
    if order not in REDUCTION_ORDERS:
        raise ValueError(f"reduction_order must be 'canonical' or 'torch', got {order!r}")
    return order


def validate_common(lr: float, betas: tuple[float, float], momentum_dtype: str, bf16_method: str,
                    foreach_batch_cutoff: int, auto_lr: bool) -> tuple[float, float]:
    beta1, beta2 = float(betas[0]), float(betas[1])
    if not 0.0 <= beta1 < 1.0:
        raise ValueError(f"betas[0] must be in [0, 1), got {beta1}")
    if not 0.0 <= beta2 < 1.0:
        raise ValueError(f"betas[1] must be in [0, 1), got {beta2}")
    if lr < 0.0:
        raise ValueError(f"lr must be >= 0, got {lr}")
    if momentum_dtype not in ("bfloat16", "float32", "int8", "4bit"):
        raise ValueError(f"momentum_dtype must be bfloat16/float32/int8/4bit, got {momentum_dtype!r}")
    if bf16_method not in ("stochastic_rounding", "kahan", "none"):
        raise ValueError(f"bf16_method must be stochastic_rounding/kahan/none, got {bf16_method!r}")
    if foreach_batch_cutoff < 1:
        raise ValueError(f"foreach_batch_cutoff must be >= 1, got {foreach_batch_cutoff}")
    if auto_lr:
        raise NotImplementedError("kaon_amd: auto_lr (the DoWG LR controller) is not part of this build")
    return beta1, beta2


class KaonOptimizer(torch.optim.Optimizer):
    """Base of the HIP-backed optimizers: plan cache, SR key, checkpoint extras.

    Subclasses provide ``_OPT`` (the C-ABI optimizer code), ``_init_state`` and
    ``_hyper``.  The SR noise key is (``sr_seed``, step count); ``sr_seed``
    defaults to ``torch.initial_seed()`` at construction, so seeding torch
    seeds the optimizer's rounding as the reference's global-RNG draw does
    (src/kaon/_stochastic_rounding.py:88-94).
    """

    _OPT = L.OPT_ADAKAON
    _NAME = "kaon"
    _HALF = False  # float16 params (RN / kahan writes, src/kaon/_backend.py:82-98)

    def __init__(self, params: Iterable[Any], defaults: dict[str, Any]) -> None:
        super().__init__(params, defaults)
        self._t = 0
        self.sr_seed = int(torch.initial_seed()) & 0xFFFFFFFF
        self._plans: dict[tuple, tuple[tuple, E.Plan]] = {}
        self._launch_cache: dict[int, tuple[tuple, list]] = {}  # param group -> (key, launches)
        self._state_version = 0
        self._inject_noise: dict[torch.Tensor, list] = {}  # tests: param -> [uint16 noise per stream]
        # After a step with gradient centralization, leave p.grad centralized as the
        # reference's path does (centralize_grads_, src/kaon/_backend.py:147-177): its
        # native paths centralize in place, its fused Adakaon / AdaPNM kernels do not.
        # One extra read and write of the 2-D gradients; set False to skip it.
        self.centralize_grads_in_place = True

    # ------------------------------------------------------------ helpers
    def _gc_writeback(self, group: dict[str, Any], plan: Any, hp: Any, dev: torch.device) -> None:
        if self.centralize_grads_in_place and group.get("gradient_centralization"):
            L.check(L.lib().kaon_gc_writeback(ctypes.byref(plan.launch), ctypes.byref(hp), E.stream_handle(dev)),
                    "kaon_gc_writeback")

    def _tensor_ids(self) -> dict[int, int]:
        return {id(p): i for i, p in enumerate(p for g in self.param_groups for p in g["params"])}

    def _invalidate(self) -> None:
        self._plans.clear()
        self._launch_cache.clear()
        self._state_version += 1

    def add_param_group(self, param_group: dict[str, Any]) -> None:
        super().add_param_group(param_group)
        if hasattr(self, "_plans"):  # tensor ids (the SR counter field) shift
            self._invalidate()

    @staticmethod
    def _stepped(group: dict[str, Any]) -> tuple[list[torch.Tensor], bytes]:
        """The group's params that have a gradient, and the pointer key of them and
        their grads (param and grad storage, grad dtype, contiguity and layout)."""
        return K.group_key(group["params"])

    def _group_key(self, group: dict[str, Any], pkey: bytes) -> tuple:
        """What a group's launches depend on: state version, codec settings, and the
        pointer key of ``_stepped``."""
        return (self._state_version, group["momentum_dtype"], group["bf16_method"], group["betas"][0] > 0, pkey)

    def _launches(self, gid: int, group: dict[str, Any], params: list[torch.Tensor], pkey: bytes) -> list:
        """The group's launches (plan, p dtype, g dtype, device, ...), reused while
        ``_group_key`` is unchanged; otherwise checks the params, creates missing state
        and plans again (``_build_launches``).  The stream is looked up per step."""
        hit = self._launch_cache.get(gid)
        if hit is not None and hit[0] == self._group_key(group, pkey):
            return hit[1]
        self._check_params(params)
        for p in params:
            state = self.state[p]
            if not state:
                self._init_state(p, state, group)
                self._state_version += 1
        out = self._build_launches(gid, group, params, self._tensor_ids())
        self._launch_cache[gid] = (self._group_key(group, pkey), out)
        return out

    def _build_launches(self, gid: int, group: dict[str, Any], params: list[torch.Tensor],
                        tids: dict[int, int]) -> list:  # pragma: no cover - abstract
        raise NotImplementedError

    def _check_params(self, params: list[torch.Tensor]) -> None:
        for p in params:
            if p.grad.is_sparse:
                raise RuntimeError(f"{self._NAME} does not support sparse gradients")
            if p.device.type != "cuda":
                raise RuntimeError(f"kaon_amd: {self._NAME} steps run on a ROCm GPU; got a param on {p.device}")
            if not p.is_contiguous():
                raise ValueError("kaon_amd: params must be contiguous")
            if p.dtype == torch.float16 or p.grad.dtype == torch.float16:
                if not self._HALF:
                    raise NotImplementedError(
                        f"kaon_amd: {self._NAME} does not step float16 params in this build (Adakaon, Lion, AdaMuon and AdaPNM do)")
                if p.dtype != p.grad.dtype:
                    raise NotImplementedError("kaon_amd: float16 params take float16 grads")
            if p.grad.dtype != p.dtype and p.grad.dtype not in (torch.float32, torch.bfloat16):
                raise NotImplementedError(f"kaon_amd: grad dtype {p.grad.dtype} is not supported")

    def _entries(self, group: dict[str, Any], params: list[torch.Tensor], tids: dict[int, int]) -> list[dict]:
        out = []
        for p in params:
            st = self.state[p]
            R, C, fac = E.matrixized(p)
            g = p.grad if p.grad.is_contiguous() else p.grad.contiguous()
            e = dict(p=p, g=g, R=R, C=C, factored=fac, tensor_id=tids[id(p)],
                     m=st.get("m"), m_scale=st.get("m_scale"), row=st.get("row"), col=st.get("col"),
                     v=st.get("v"), shift=st.get("shift"), block4=st.get("m_block", 0),
                     noise=self._inject_noise.get(p))
            out.append(e)
        return out

    def _plan(self, key: tuple, group: dict[str, Any], params: list[torch.Tensor], codec: int,
              tids: dict[int, int], opt: int | None = None) -> E.Plan:
        opt = self._OPT if opt is None else opt
        method = L.BF16_METHOD[group["bf16_method"]]
        ptrs = (self._state_version, codec, method, opt) + tuple(
            (p.data_ptr(), p.grad.data_ptr()) for p in params)
        hit = self._plans.get(key)
        if hit is not None and hit[0] == ptrs:
            return hit[1]
        for p in params:
            if not p.grad.is_contiguous():
                raise ValueError("kaon_amd: gradients must be contiguous")
        plan = E.Plan(opt, codec, self._entries(group, params, tids), params[0].device,
                      E.dtype_code(params[0].dtype), E.dtype_code(params[0].grad.dtype), method)
        self._plans[key] = (ptrs, plan)
        return plan

    def _partitions(self, params: list[torch.Tensor]) -> dict[tuple[int, int], list[torch.Tensor]]:
        parts: dict[tuple[int, int], list[torch.Tensor]] = {}
        for p in params:
            parts.setdefault((E.dtype_code(p.dtype), E.dtype_code(p.grad.dtype)), []).append(p)
        return parts

    # ------------------------------------------------------------ checkpoint
    def state_dict(self) -> dict[str, Any]:
        sd = super().state_dict()
        sd["kaon_amd"] = {"step": self._t, "sr_seed": self.sr_seed}
        return sd

    def load_state_dict(self, state_dict: dict[str, Any]) -> None:
        sd = dict(state_dict)
        extra = sd.pop("kaon_amd", None)
        sd.pop("_autolr", None)
        load_state_dict_preserving_dtypes(self, sd)
        if extra is not None:
            self._t = int(extra.get("step", self._t))
            self.sr_seed = int(extra.get("sr_seed", self.sr_seed))
        self._invalidate()

    def step(self, *args: Any, **kwargs: Any) -> Any:
        """One optimizer step; ``closure`` optional, as torch.optim's.

        torch.optim.Optimizer wraps a subclass's ``step`` in a profiler range
        and the step hooks unless the method is marked ``hooked``.  This one is:
        it runs the same hooks in the same order (the global then the instance
        pre-hooks, which may replace the arguments; the step; the instance then
        the global post-hooks) and opens the same profiler range, but only while
        a profiler is active.  The wrapper's range costs as much host time as the
        rest of a step over a bag of small tensors."""
        if torch.autograd._profiler_enabled():
            with torch.autograd.profiler.record_function(f"Optimizer.step#{type(self).__name__}.step"):
                return self._hooked_step(args, kwargs)
        return self._hooked_step(args, kwargs)

    step.hooked = True  # type: ignore[attr-defined]

    def _hooked_step(self, args: tuple, kwargs: dict) -> Any:
        a = (self,) + tuple(args)
        pre, post = self._optimizer_step_pre_hooks, self._optimizer_step_post_hooks
        gpre, gpost = _topt._global_optimizer_pre_hooks, _topt._global_optimizer_post_hooks
        if pre or gpre:
            for hook in chain(gpre.values(), pre.values()):
                result = hook(self, a, kwargs)
                if result is not None:
                    if isinstance(result, tuple) and len(result) == 2:
                        a, kwargs = result
                    else:
                        raise RuntimeError(f"{self.step} must return None or a tuple of (new_args, new_kwargs), "
                                           f"but got {result}.")
        out = self._step_impl(*a[1:], **kwargs)
        self._optimizer_step_code()
        if post or gpost:
            for hook in chain(post.values(), gpost.values()):
                hook(self, a, kwargs)
        return out

    def _step_impl(self, closure: Any = None, nk: Any = None) -> Any:  # pragma: no cover - abstract
        raise NotImplementedError
