"""Plans and launches: the host side of the multi-tensor descriptor table.

One :class:`Plan` covers the params of one param group that share (param
dtype, grad dtype).  It holds the device copy of the descriptor table and the
work-item tables that ``kaon_plan`` (C++) produced, plus the workspace.  Plans
are cached by the optimizer and rebuilt when any param or grad pointer changes
(the stale-pointer hazard the reference guards against in
src/kaon/_fused_triton.py:1229-1245), when state is (re)initialized or loaded.
"""
from __future__ import annotations

import ctypes
import math
from typing import Any, Sequence

import torch

from . import _lib as L


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return L.BF16
    if dt == torch.float32:
        return L.F32
    if dt == torch.float16:
        return L.F16
    raise NotImplementedError(
        f"kaon_amd: params/grads of dtype {dt} are not supported (bfloat16, float16 and float32 are)")


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _align(n: int, a: int = 256) -> int:
    return (n + a - 1) // a * a


_MOM_DTYPE = {L.MOM_F32: torch.float32, L.MOM_BF16: torch.bfloat16, L.MOM_INT8: torch.int8,
              L.MOM_4BIT: torch.uint8}


def _check_state(e: dict[str, Any], codec: int, i: int) -> None:
    """The state tensors of entry ``e`` hold what the kernels will read and write for
    ``codec``: a momentum buffer (and its scales) of the codec's dtype and size, and
    second-moment buffers of the param's matrixized shape.  State created for another
    ``momentum_dtype`` or ``betas`` (the group changed after the first step) or loaded
    for another shape raises here instead of being overrun on the device."""
    p = e["p"]
    n, R, C = p.numel(), e["R"], e["C"]

    def bad(key: str, why: str) -> None:
        raise ValueError(f"kaon_amd: param {i} {tuple(p.shape)}: state '{key}' {why}; the state does not match "
                         "the group's settings (momentum_dtype / betas changed after the state was created, or "
                         "a checkpoint of another shape was loaded)")

    def need(key: str, t: torch.Tensor | None, dtype: torch.dtype, numel: int) -> None:
        if t is None:
            bad(key, "is missing")
        if t.dtype != dtype:
            bad(key, f"has dtype {t.dtype}, expected {dtype}")
        if t.numel() != numel:
            bad(key, f"has {t.numel()} elements, expected {numel}")
        if not t.is_contiguous() or t.device != p.device:
            bad(key, "must be a contiguous tensor on the param's device")

    for key, skey in (("m", "m_scale"), ("m2", "m2_scale")):
        if key == "m2" and e.get("m2") is None:
            continue
        if codec == L.MOM_NONE:
            continue
        m = e.get(key)
        if codec == L.MOM_4BIT:
            need(key, m, torch.uint8, (n + 1) // 2)
            blk = int(e.get("block4", 0))
            if blk < 1:
                bad(key, "has no 4-bit block size")
            need(skey, e.get(skey), torch.float32, (n + blk - 1) // blk)
        else:
            need(key, m, _MOM_DTYPE[codec], n)
            if codec == L.MOM_INT8:
                need(skey, e.get(skey), torch.float32, R if e["factored"] else 1)
    fb_r, fb_c = e.get("fb", (0, 0))
    rows, cols = (n // fb_c, n // fb_r) if fb_r else (R, C)
    for key, numel in (("row", rows), ("col", cols), ("v", n), ("max_v", n)):
        t = e.get(key)
        if t is not None:
            need(key, t, torch.float32, numel)


class Plan:
    """Device tables + workspace of one planned launch group."""

    def __init__(self, opt: int, codec: int, entries: Sequence[dict[str, Any]], device: torch.device,
                 p_dtype: int = L.BF16, g_dtype: int = L.BF16, bf16_method: int = L.SR) -> None:
        n = len(entries)
        for i, e in enumerate(entries):
            _check_state(e, codec, i)
        descs = (L.KaonTensor * max(n, 1))()
        for i, e in enumerate(entries):
            d = descs[i]
            d.g, d.p = _ptr(e["g"]), _ptr(e["p"])
            d.m, d.m_scale = _ptr(e.get("m")), _ptr(e.get("m_scale"))
            d.row, d.col, d.v = _ptr(e.get("row")), _ptr(e.get("col")), _ptr(e.get("v"))
            d.shift = _ptr(e.get("shift"))
            d.m2, d.m2_scale, d.max_v = _ptr(e.get("m2")), _ptr(e.get("m2_scale")), _ptr(e.get("max_v"))
            if e.get("pd_s") is not None:
                d.pd_s, d.pd_p0 = _ptr(e["pd_s"]), _ptr(e["pd_p0"])
                d.pd_ns, d.pd_slice = e["pd_s"].numel(), int(e["pd_slice"])
                d.pd_p0_scalar = 1 if e["pd_p0"].dim() == 0 else 0
                d.full_v = 1 if e.get("full_v") else 0
            noise = e.get("noise") or (None, None, None)
            for s in range(3):
                d.noise[s] = _ptr(noise[s])
            d.R, d.C = e["R"], e["C"]
            d.factored = 1 if e["factored"] else 0
            d.block4 = int(e.get("block4", 0))
            d.tensor_id = int(e["tensor_id"])
            d.gc_write = 1 if e.get("gc_write", True) else 0
            d.fb_r, d.fb_c = e.get("fb", (0, 0))
        # whether a launch with KAON_F_GC_WRITE would store any tensor's gradient
        self.any_gc_write = any(e.get("gc_write", True) and e["factored"] for e in entries)
        # whether a tensor's second moment is factored over its last two dims (KProdigy)
        self.any_fb = any(e.get("fb") for e in entries)
        info = L.KaonPlanInfo()
        args = L.KaonPlanArgs(opt, codec, p_dtype, g_dtype, bf16_method)
        lib = L.lib()
        L.check(lib.kaon_plan(ctypes.byref(args), descs, n, None, None, None, None, None, None,
                              ctypes.byref(info)), "kaon_plan")
        rows = (L.KaonItem * max(info.n_row_items, 1))()
        elems = (L.KaonItem * max(info.n_elem_items, 1))()
        fins = (L.KaonItem * max(info.n_fin_items, 1))()
        flats = (L.KaonItem * max(info.n_flat_items, 1))()
        nsq = (L.KaonItem * max(info.n_ns_sq, 1))()
        nrect = (L.KaonItem * max(info.n_ns_rect, 1))()
        L.check(lib.kaon_plan(ctypes.byref(args), descs, n, rows, elems, fins, flats, nsq, nrect,
                              ctypes.byref(info)), "kaon_plan")
        self.info = info
        self.descs = descs
        parts = [bytes(descs)[: ctypes.sizeof(L.KaonTensor) * n],
                 bytes(rows)[: 16 * info.n_row_items],
                 bytes(elems)[: 16 * info.n_elem_items],
                 bytes(fins)[: 16 * info.n_fin_items],
                 bytes(flats)[: 16 * info.n_flat_items],
                 bytes(nsq)[: 16 * info.n_ns_sq],
                 bytes(nrect)[: 16 * info.n_ns_rect]]
        offs, total = [], 0
        for b in parts:
            offs.append(total)
            total += _align(max(len(b), 1))
        blob = bytearray(total)
        for o, b in zip(offs, parts):
            blob[o:o + len(b)] = b
        self.table = torch.frombuffer(blob, dtype=torch.uint8).to(device)
        self.workspace = torch.empty(max(int(info.ws_words), 4), dtype=torch.float32, device=device)
        base = self.table.data_ptr()
        la = L.KaonLaunch()
        (la.descs, la.row_items, la.elem_items, la.fin_items, la.flat_items, la.ns_sq_items,
         la.ns_rect_items) = (base + o for o in offs)
        la.n_tensors, la.n_row_items = n, info.n_row_items
        la.n_fin_items, la.n_flat_items = info.n_fin_items, info.n_flat_items
        for k in range(L.ROW_CLASSES):
            la.row_runs[k] = info.row_runs[k]
        la.n_fast, la.n_elem_items = info.n_fast, info.n_elem_items
        la.n_ns_sq, la.n_ns_rect = info.n_ns_sq, info.n_ns_rect
        la.n_ns_sq_big, la.n_ns_rect_big = info.n_ns_sq_big, info.n_ns_rect_big
        la.workspace = self.workspace.data_ptr()
        la.ws_words = int(info.ws_words)
        la.n_long, la.n_long_fast, la.n_long_rest = info.n_long, info.n_long_fast, info.n_long_rest
        self.launch = la


def matrixized(p: torch.Tensor) -> tuple[int, int, bool]:
    """(R, C, factored): ndim >= 2 -> [shape[0], numel/shape[0]] (conv matrixized,
    src/kaon/adakaon.py:975-981); otherwise one row of numel elements."""
    if p.ndim >= 2:
        r = int(p.shape[0])
        return r, (p.numel() // r if r else 0), True
    return 1, p.numel(), False


def f32(x: float) -> float:
    """Round a python float to fp32 as torch does for a scalar operand."""
    return float(torch.tensor(x, dtype=torch.float32).item()) if math.isfinite(x) else x
