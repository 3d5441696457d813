"""CPU parity oracle for the kaon fused optimizer step.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this module, and only as the
checker (or as the timed CPU baseline); the product path
(``k-optimizers_amd/kaon_amd``) never imports it and fails loudly without its
HIP library.

This wraps ``kaon_oracle.c`` (the per-tensor restatement of the reference
step, see the header of that file for the reference citations and the
rounding / reduction-order model) with numpy state that mirrors the
reference's per-parameter state layout:

* Adakaon ``_init_state``  -- src/kaon/adakaon.py:318-335
* Lion ``_init_state``     -- src/kaon/lion.py:210-241
* AdaMuon ``_init_state``  -- src/kaon/adamuon.py:297-316
* codec ``init_state``     -- src/kaon/_momentum_codec.py:263-264, 296-301, 351-361
* MSAM / Nekaon lookahead  -- src/kaon/msam.py:169-188, 375-406; src/kaon/nekaon.py:162-171
* AdaPNM ``_init_state`` / ``_alloc_momentum`` -- src/kaon/adapnm.py:451-500 (two momenta,
  ``m_pos`` / ``m_neg``, whose roles alternate by step parity, :588-596)
* KProdigy ``_init_state`` / ``_step_scope`` -- src/kaon/kprodigy.py:262-291, 306-386 (the D
  update folds the per-tensor statistics in param order in fp32, then runs in double)

Arrays: bf16 tensors are ``np.uint16`` bit patterns, fp32 are ``np.float32``.

How it is pinned (tests/):

* the reference's own output on seeded inputs with the oracle's SR noise
  injected (``tests/golden/``, written by ``tests/golden/make_golden.py``):
  every optimizer above, bit-exact up to torch's unspecified fp32 reduction
  order (``test_oracle_golden.py``); KProdigy also per-step D; MSAM's global
  norm from the reference's per-step momentum, and its step with the
  reference's norms fed in (``mnorm_feed``), bit-exact;
* known answers and closed forms: Philox4x32-10 vectors, the SR bit trick,
  the int8 / 4-bit codecs, CSUM (``test_oracle_kat.py``);
* torch-CPU arithmetic it mirrors: lerp, add_/addcmul_ fma forms, bf16 GC
  (``test_oracle_torch_semantics.py``).

Parity unpinned: NaN payload bits (positions are compared).
"""
from __future__ import annotations

import contextlib
import ctypes
import math
import os
from dataclasses import dataclass, field
from typing import Any

import numpy as np

F32, BF16, F16 = 0, 1, 2
MOM_CODE = {"none": 0, "float32": 1, "bfloat16": 2, "int8": 3, "4bit": 4}
BF16_METHOD = {"stochastic_rounding": 0, "none": 1, "kahan": 2}

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")


class KoTensor(ctypes.Structure):
    _fields_ = [
        ("g", ctypes.c_void_p), ("p", ctypes.c_void_p), ("m", ctypes.c_void_p),
        ("m_scale", ctypes.c_void_p), ("row", ctypes.c_void_p), ("col", ctypes.c_void_p),
        ("v", ctypes.c_void_p), ("shift", ctypes.c_void_p),
        ("R", ctypes.c_int64), ("C", ctypes.c_int64),
        ("g_dtype", ctypes.c_int32), ("p_dtype", ctypes.c_int32),
        ("codec", ctypes.c_int32), ("block4", ctypes.c_int32),
        ("factored", ctypes.c_int32), ("tensor_id", ctypes.c_uint32),
        ("noise", ctypes.c_void_p * 3),
        ("out_m", ctypes.c_void_p),
        ("fac_override", ctypes.c_void_p),
        ("m2", ctypes.c_void_p), ("m2_scale", ctypes.c_void_p), ("max_v", ctypes.c_void_p),
        ("pd_s", ctypes.c_void_p), ("pd_p0", ctypes.c_void_p), ("pd_np0", ctypes.c_int64),
        ("pd_slice", ctypes.c_int32), ("full_v", ctypes.c_int32),
        ("torch_order", ctypes.c_int32),
        ("ss_out", ctypes.c_void_p),
        ("fb_r", ctypes.c_int64), ("fb_c", ctypes.c_int64),
    ]


class KoHyper(ctypes.Structure):
    _fields_ = [
        ("lr", ctypes.c_double), ("beta1", ctypes.c_double), ("beta2", ctypes.c_double),
        ("eps1", ctypes.c_double), ("wd", ctypes.c_double), ("clip", ctypes.c_double),
        ("cautious", ctypes.c_int32), ("gc", ctypes.c_int32), ("bf16_method", ctypes.c_int32),
        ("ns_steps", ctypes.c_int32),
        ("seed", ctypes.c_uint64), ("step", ctypes.c_uint32),
        ("nk_remove", ctypes.c_int32), ("nk_climb", ctypes.c_int32),
        ("nk_k", ctypes.c_double), ("nk_bound_old", ctypes.c_double), ("nk_bound_new", ctypes.c_double),
        ("beta0", ctypes.c_double), ("ams_bound", ctypes.c_int32),
        ("pd_d", ctypes.c_double), ("pd_dlr", ctypes.c_double), ("pd_alpha_s", ctypes.c_double),
        ("pd_beta3", ctypes.c_double), ("pd_eps", ctypes.c_double),
        ("pd_decouple", ctypes.c_int32), ("pd_stats", ctypes.c_int32),
    ]


_lib_handle = None


def lib() -> ctypes.CDLL:
    """The compiled oracle (``make -C oracle``; ``__graft_entry__.build()`` runs it)."""
    global _lib_handle
    if _lib_handle is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run `make -C oracle`)")
        L = ctypes.CDLL(_LIB_PATH)
        for name in ("ko_adakaon_tensor", "ko_lion_tensor", "ko_adamuon_tensor", "ko_adapnm_tensor"):
            getattr(L, name).argtypes = [ctypes.POINTER(KoTensor), ctypes.POINTER(KoHyper)]
            getattr(L, name).restype = ctypes.c_int
        L.ko_kprodigy_pass1_tensor.argtypes = [ctypes.POINTER(KoTensor), ctypes.POINTER(KoHyper),
                                               ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float)]
        L.ko_kprodigy_pass1_tensor.restype = ctypes.c_int
        L.ko_kprodigy_pass2_tensor.argtypes = [ctypes.POINTER(KoTensor), ctypes.POINTER(KoHyper)]
        L.ko_kprodigy_pass2_tensor.restype = ctypes.c_int
        L.ko_momentum_sumsq.argtypes = [ctypes.POINTER(KoTensor)]
        L.ko_momentum_sumsq.restype = ctypes.c_float
        L.ko_fsum.argtypes = [ctypes.c_void_p, ctypes.c_int64]
        L.ko_fsum.restype = ctypes.c_float
        L.ko_msam_apply.argtypes = [ctypes.POINTER(KoTensor), ctypes.POINTER(KoHyper),
                                    ctypes.c_double, ctypes.c_double, ctypes.c_uint32]
        for name in ("ko_f32_to_f16", "ko_f16_to_f32"):
            getattr(L, name).argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
            getattr(L, name).restype = None
        L.ko_csum.argtypes = [ctypes.c_void_p, ctypes.c_int64]
        L.ko_csum.restype = ctypes.c_float
        for name in ("ko_torch_inner_sum", "ko_torch_sumsq"):
            getattr(L, name).argtypes = [ctypes.c_void_p, ctypes.c_int64]
            getattr(L, name).restype = ctypes.c_float
        L.ko_torch_outer_sum.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
        L.ko_torch_outer_sum.restype = None
        L.ko_rows_per_wave.argtypes = [ctypes.c_int64]
        L.ko_rows_per_wave.restype = ctypes.c_int64
        L.ko_philox4x32_10.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        L.ko_sr_noise_fill.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint64,
                                       ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]
        L.ko_quant_int8.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                    ctypes.c_void_p, ctypes.c_void_p]
        L.ko_quant_4bit.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32,
                                    ctypes.c_void_p, ctypes.c_void_p]
        L.ko_dequant.argtypes = [ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                 ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p]
        L.ko_sr_round.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
        L.ko_newton_schulz.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                       ctypes.c_int32, ctypes.c_void_p]
        L.ko_vec_lerp.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float, ctypes.c_int64,
                                  ctypes.c_void_p]
        L.ko_vec_gc_bf16.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
        _lib_handle = L
    return _lib_handle


def _ptr(a: np.ndarray | None) -> int | None:
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ------------------------------------------------------------------ bf16 helpers
def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even, NaN -> 0x7FC0.

    u + 0x7FFF + lsb fits in 32 bits for every non-NaN pattern (the largest,
    0xFF7FFFFF + 0x8000, rounds to -inf); only negative NaNs wrap, and they are
    replaced below."""
    u = np.ascontiguousarray(x, dtype=np.float32).reshape(-1).view(np.uint32)
    t = (u >> 16) & np.uint32(1)
    t += u
    t += np.uint32(0x7FFF)
    t >>= 16
    r = t.astype(np.uint16)
    r[(u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)] = 0x7FC0
    return r.reshape(np.shape(x))


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    """fp32 -> binary16 bits, round to nearest even, overflow to inf, NaN -> 0x7E00
    with the sign (kaon_oracle.c f_to_f16)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().ko_f32_to_f16(_ptr(x), x.size, _ptr(out))
    return out


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().ko_f16_to_f32(_ptr(h), h.size, _ptr(out))
    return out


# ------------------------------------------------------------------ primitives
def csum(x: np.ndarray) -> np.float32:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return np.float32(lib().ko_csum(_ptr(x), x.size))


def torch_inner_sum(x: np.ndarray) -> np.float32:
    """torch CPU's fp32 sum of a contiguous row (ko_torch_inner_sum)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    return np.float32(lib().ko_torch_inner_sum(_ptr(x), x.size))


def torch_outer_sum(x: np.ndarray) -> np.ndarray:
    """torch CPU's fp32 sums over the rows of a contiguous [R, C] matrix (ko_torch_outer_sum)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    R, C = x.shape
    out = np.zeros(C, dtype=np.float32)
    lib().ko_torch_outer_sum(_ptr(x), R, C, _ptr(out))
    return out


def torch_sumsq(x: np.ndarray) -> np.float32:
    """torch CPU's fp32 sum of squares inside t.norm(2) (ko_torch_sumsq)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    return np.float32(lib().ko_torch_sumsq(_ptr(x), x.size))


@contextlib.contextmanager
def torch_order():
    """Within the block every oracle step sums in torch CPU's order (tests only)."""
    TORCH_ORDER[0] = True
    try:
        yield
    finally:
        TORCH_ORDER[0] = False


def rows_per_wave(C: int) -> int:
    """Rows per wave group of the canonical column-sum order."""
    return int(lib().ko_rows_per_wave(C))


def philox4x32_10(ctr, key) -> np.ndarray:
    c = np.asarray(ctr, dtype=np.uint32).copy()
    k = np.asarray(key, dtype=np.uint32).copy()
    out = np.zeros(4, dtype=np.uint32)
    lib().ko_philox4x32_10(_ptr(c), _ptr(k), _ptr(out))
    return out


def sr_noise(n: int, seed: int, step: int, tensor_id: int, stream: int) -> np.ndarray:
    out = np.zeros(max(n, 1), dtype=np.uint16)
    lib().ko_sr_noise_fill(_ptr(out), n, seed, step, tensor_id, stream)
    return out[:n]


def sr_round(x: np.ndarray, noise: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    noise = np.ascontiguousarray(noise, dtype=np.uint16)
    out = np.zeros(x.size, dtype=np.uint16)
    lib().ko_sr_round(_ptr(x), _ptr(noise), x.size, _ptr(out))
    return out.reshape(x.shape)


def quant_int8(m: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """_quant_int8 (src/kaon/_momentum_codec.py:72-83): per-row for ndim>=2, scalar for 1-D."""
    m = np.ascontiguousarray(m, dtype=np.float32)
    rows = m.shape[0] if m.ndim >= 2 else 1
    cols = m.size // max(rows, 1)
    q = np.zeros(m.shape, dtype=np.int8)
    sc = np.zeros(rows, dtype=np.float32)
    lib().ko_quant_int8(_ptr(m), rows, cols, _ptr(q), _ptr(sc))
    return q, sc


def quant_4bit(m: np.ndarray, block: int) -> tuple[np.ndarray, np.ndarray]:
    """_quant_4bit (src/kaon/_momentum_codec.py:122-141)."""
    m = np.ascontiguousarray(m, dtype=np.float32).reshape(-1)
    n = m.size
    nb = (n + block - 1) // block
    pk = np.zeros((n + 1) // 2, dtype=np.uint8)
    sc = np.zeros(nb, dtype=np.float32)
    lib().ko_quant_4bit(_ptr(m), n, block, _ptr(pk), _ptr(sc))
    return pk, sc


def dequant(codec: str, m: np.ndarray, scale: np.ndarray | None, shape, block: int = 0) -> np.ndarray:
    n = int(np.prod(shape)) if len(shape) else 1
    rows = shape[0] if len(shape) >= 2 else 1
    cols = n // max(rows, 1)
    out = np.zeros(max(n, 1), dtype=np.float32)
    lib().ko_dequant(MOM_CODE[codec], _ptr(np.ascontiguousarray(m)),
                     _ptr(None if scale is None else np.ascontiguousarray(scale, dtype=np.float32)),
                     rows, cols, block, _ptr(out))
    return out[:n].reshape(shape)


def lerp(a: np.ndarray, b: np.ndarray, w: float) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    out = np.zeros_like(a)
    lib().ko_vec_lerp(_ptr(a), _ptr(b), float(np.float32(w)), a.size, _ptr(out))
    return out


def gc_bf16(g_bits: np.ndarray) -> np.ndarray:
    """Gradient centralization of a bf16 [R, C] array (bits), in the grad dtype."""
    g = np.ascontiguousarray(g_bits, dtype=np.uint16)
    R = g.shape[0]
    C = g.size // R
    out = np.zeros_like(g)
    lib().ko_vec_gc_bf16(_ptr(g), R, C, _ptr(out))
    return out


def newton_schulz(x: np.ndarray, steps: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros_like(x)
    lib().ko_newton_schulz(_ptr(x), x.shape[0], x.shape[1], steps, _ptr(out))
    return out


# ------------------------------------------------------------------ parameters
def fourbit_block_size(numel: int, bs: int) -> int:
    """src/kaon/_momentum_codec.py:192-200."""
    return numel if bs <= 0 else (min(bs, numel) if numel > 0 else 1)


@dataclass
class OParam:
    """One parameter, its gradient and its optimizer state, as numpy arrays."""

    p: np.ndarray                 # uint16 (bf16 bits) or float32, param shape
    p_dtype: int
    shape: tuple[int, ...]
    tensor_id: int = 0
    g: np.ndarray | None = None   # uint16 or float32, param shape
    g_dtype: int = BF16
    state: dict[str, Any] = field(default_factory=dict)

    @property
    def numel(self) -> int:
        return int(np.prod(self.shape)) if len(self.shape) else 1

    @property
    def factored(self) -> bool:
        return len(self.shape) >= 2

    @property
    def eff(self) -> tuple[int, int]:
        if self.factored:
            return self.shape[0], self.numel // self.shape[0]
        return 1, self.numel


def _alloc_momentum(st: dict[str, Any], prefix: str, prm: OParam, group: dict[str, Any]) -> None:
    """One momentum buffer under ``prefix`` (src/kaon/adapnm.py:451-479; the codec
    layouts of src/kaon/_momentum_codec.py:263-264, 296-301, 351-361)."""
    R, _ = prm.eff
    n = prm.numel
    md = group["momentum_dtype"]
    if md == "float32":
        st[prefix] = np.zeros(prm.shape, dtype=np.float32)
    elif md == "bfloat16":
        st[prefix] = np.zeros(prm.shape, dtype=np.uint16)
    elif md == "int8":
        st[prefix] = np.zeros(prm.shape, dtype=np.int8)
        st[f"{prefix}_scale"] = np.ones(R if prm.factored else 1, dtype=np.float32)
    else:
        bs = fourbit_block_size(n, group["momentum_4bit_block"])
        st[prefix] = np.full((n + 1) // 2, 0x88, dtype=np.uint8)
        st[f"{prefix}_scale"] = np.ones((n + bs - 1) // bs, dtype=np.float32)
        st[f"{prefix}_numel"] = n
        st[f"{prefix}_block"] = bs


def init_state(prm: OParam, opt: str, group: dict[str, Any]) -> None:
    st = prm.state
    R, C = prm.eff
    n = prm.numel
    if opt == "kprodigy":
        # src/kaon/kprodigy.py:262-291
        sliced = values(prm.p, prm.p_dtype).reshape(-1)[:: group["slice_p"]].astype(np.float32)
        st["step"] = 0
        st["s"] = np.zeros(sliced.size, dtype=np.float32)
        st["p0"] = sliced.copy() if float(np.sqrt(np.sum(sliced.astype(np.float64) ** 2))) > 0 else \
            np.zeros((), dtype=np.float32)
        if group["betas"][0] > 0:
            _alloc_momentum(st, "m", prm, group)
        if group["second_moment"] == "factored" and prm.factored:
            if len(prm.shape) > 2 and not group.get("factor_conv_as_matrix", True):
                # factored over the last two dims (kprodigy.py:286-288)
                st["row"] = np.zeros(prm.shape[:-1], dtype=np.float32)
                st["col"] = np.zeros(prm.shape[:-2] + prm.shape[-1:], dtype=np.float32)
            else:
                st["row"] = np.zeros(R, dtype=np.float32)
                st["col"] = np.zeros(C, dtype=np.float32)
        else:
            st["v"] = np.zeros(prm.shape, dtype=np.float32)
        if prm.p_dtype in (BF16, F16) and group.get("bf16_method") == "kahan":
            st["shift"] = np.zeros(prm.shape, dtype=np.uint16)
        return
    if opt == "adapnm":
        if prm.factored:
            st["row"] = np.zeros(R, dtype=np.float32)
            st["col"] = np.zeros(C, dtype=np.float32)
        else:
            st["v"] = np.zeros(n, dtype=np.float32)
            if group.get("ams_bound"):
                st["max_v"] = np.zeros(n, dtype=np.float32)
        _alloc_momentum(st, "m_pos", prm, group)
        _alloc_momentum(st, "m_neg", prm, group)
        if prm.p_dtype in (BF16, F16) and group.get("bf16_method") == "kahan":
            st["shift"] = np.zeros(prm.shape, dtype=np.uint16)
        return
    if opt in ("adakaon", "adamuon"):
        if prm.factored:
            st["row"] = np.zeros(R, dtype=np.float32)
            st["col"] = np.zeros(C, dtype=np.float32)
        else:
            st["v"] = np.zeros(n, dtype=np.float32)
    md = group["momentum_dtype"]
    if group["betas"][0] > 0 or opt == "lion":
        if md == "float32":
            st["m"] = np.zeros(prm.shape, dtype=np.float32)
        elif md == "bfloat16":
            st["m"] = np.zeros(prm.shape, dtype=np.uint16)
        elif md == "int8":
            st["m"] = np.zeros(prm.shape, dtype=np.int8)
            st["m_scale"] = np.ones(R if prm.factored else 1, dtype=np.float32)
        else:
            bs = fourbit_block_size(n, group["momentum_4bit_block"])
            st["m"] = np.full((n + 1) // 2, 0x88, dtype=np.uint8)
            st["m_scale"] = np.ones((n + bs - 1) // bs, dtype=np.float32)
            st["m_numel"] = n
            st["m_block"] = bs
    if prm.p_dtype in (BF16, F16) and group.get("bf16_method") == "kahan":
        st["shift"] = np.zeros(prm.shape, dtype=np.uint16)


# Tests only: TORCH_ORDER[0] = True makes every tensor of the following steps sum
# in torch CPU's order (KoTensor.torch_order) instead of the canonical one.
TORCH_ORDER = [False]


def _tensor(prm: OParam, codec: str, noise=None, out_m=None, fac_override=None, ss_out=None) -> KoTensor:
    st = prm.state
    R, C = prm.eff
    t = KoTensor()
    t.g = _ptr(prm.g)
    t.p = _ptr(prm.p)
    t.m = _ptr(st.get("m"))
    t.m_scale = _ptr(st.get("m_scale"))
    t.row = _ptr(st.get("row"))
    t.col = _ptr(st.get("col"))
    t.v = _ptr(st.get("v"))
    t.shift = _ptr(st.get("shift"))
    t.R, t.C = R, C
    t.g_dtype, t.p_dtype = prm.g_dtype, prm.p_dtype
    t.codec = MOM_CODE[codec] if "m" in st else 0
    t.block4 = int(st.get("m_block", 0))
    t.factored = int(prm.factored)
    t.tensor_id = prm.tensor_id
    if noise is not None:
        for s in range(3):
            if noise[s] is not None:
                t.noise[s] = _ptr(noise[s])
    t.out_m = _ptr(out_m)
    t.fac_override = _ptr(fac_override)
    t.torch_order = int(TORCH_ORDER[0])
    t.ss_out = _ptr(ss_out)
    return t


def _pd_tensor(prm: OParam, group: dict[str, Any], noise=None) -> KoTensor:
    st = prm.state
    t = _tensor(prm, group["momentum_dtype"], noise)
    t.pd_s = _ptr(st["s"])
    p0 = st["p0"]
    if p0.ndim == 0:
        st["_p0_1"] = p0.reshape(1).copy()
        t.pd_p0, t.pd_np0 = _ptr(st["_p0_1"]), 1
    else:
        t.pd_p0, t.pd_np0 = _ptr(p0), p0.size
    t.pd_slice = int(group["slice_p"])
    t.full_v = int("v" in st)
    if "row" in st and st["row"].ndim > 1:  # factored over the last two dims
        t.fb_r, t.fb_c = prm.shape[-2], prm.shape[-1]
    return t


def _pnm_tensor(prm: OParam, codec: str, step: int, noise=None) -> KoTensor:
    """AdaPNM: m = this step's positive buffer, m2 = the negative one
    (_pos_neg_prefixes, src/kaon/adapnm.py:588-596: m_pos on odd steps)."""
    st = prm.state
    pos, neg = ("m_pos", "m_neg") if step % 2 == 1 else ("m_neg", "m_pos")
    t = _tensor(prm, codec, noise)
    t.m, t.m_scale = _ptr(st[pos]), _ptr(st.get(f"{pos}_scale"))
    t.m2, t.m2_scale = _ptr(st[neg]), _ptr(st.get(f"{neg}_scale"))
    t.max_v = _ptr(st.get("max_v"))
    t.codec = MOM_CODE[codec]
    t.block4 = int(st.get("m_pos_block", 0))
    return t


def _hyper(group: dict[str, Any], seed: int, step: int) -> KoHyper:
    h = KoHyper()
    h.lr = group["lr"]
    h.beta1, h.beta2 = group["betas"]
    eps = group.get("eps", (0.0, 0.0))
    h.eps1 = eps if isinstance(eps, float) else eps[0]
    h.wd = group.get("weight_decay", 0.0)
    h.clip = group.get("clip_threshold", 1.0)
    h.cautious = int(group.get("cautious", True))
    h.gc = int(group.get("gradient_centralization", True))
    h.bf16_method = BF16_METHOD[group.get("bf16_method", "stochastic_rounding")]
    h.ns_steps = int(group.get("ns_steps", 2))
    h.seed = seed
    h.step = step
    h.beta0 = float(group.get("beta0", 0.0))
    h.ams_bound = int(bool(group.get("ams_bound", False)))
    return h


def _check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(f"oracle returned {rc}")


class OracleOptimizer:
    """Step driver over a list of OParam for one param group.

    ``opt`` is ``"adakaon" | "lion" | "adamuon" | "nekaon" | "adapnm" | "kprodigy"``.  Nekaon is the MSAM
    ``norm="none"``, ``rho=-k`` preset over Adakaon (src/kaon/nekaon.py:162-171):
    the removal of the previous climb and the new climb are folded into the
    per-tensor step exactly where MSAM.step runs them (msam.py:384-403).
    """

    def __init__(self, params: list[OParam], opt: str, group: dict[str, Any], seed: int = 0) -> None:
        self.params = params
        self.opt = opt
        self.group = dict(group)
        self.seed = seed
        self.t = 0
        self.has_e = False
        self.bound = 0.0   # frozen climb bound (msam.py:169-188)
        self.k = float(group.get("k", 0.0))
        self.mnorm = 0.0   # MSAM norm="global": ||m|| cached at climb time
        self.mnorm_log: list[float] = []           # the norm this oracle computed, per step
        self.mnorm_feed: list[float] | None = None  # tests: norms to use instead (another sum order)
        self.rho, self.norm, self.meps = -self.k, "none", 1e-12
        if opt == "msam":  # MSAM(norm=...) over Adakaon; norm "none" is Nekaon's rho = -k form
            self.rho, self.norm, self.meps = float(group["rho"]), group["norm"], float(group.get("msam_eps", 1e-12))
            self.k = -self.rho
        for prm in params:
            init_state(prm, "adakaon" if opt in ("nekaon", "msam") else opt, self.group)

    def _kprodigy_step(self, noise: dict[int, list] | None) -> None:
        """KProdigy._step_scope (src/kaon/kprodigy.py:306-386) for one group."""
        g = self.group
        beta1, beta2 = g["betas"]
        beta3 = g["beta3"] if g.get("beta3") is not None else math.sqrt(beta2)
        k, d, d_max, d0 = g["k"], g["d"], g["d_max"], g["d0"]
        lr = g["lr"]
        bias_correction = (((1 - beta2 ** (k + 1)) ** 0.5) / (1 - beta1 ** (k + 1))
                           if g["use_bias_correction"] else 1.0)
        dlr = d * lr * bias_correction
        should_update_d = (k % g["d_update_freq"]) == 0
        d_over_d0 = d / d0
        d_numerator = g["d_numerator"] * beta3
        stats = lr > 0.0 and should_update_d
        h = _hyper(g, self.seed, self.t)
        h.eps1 = g["eps_factored"]
        h.pd_d, h.pd_dlr, h.pd_beta3, h.pd_eps = d, dlr, beta3, g["eps"]
        h.pd_alpha_s = d_over_d0 * d if g["safeguard_warmup"] else d_over_d0 * dlr
        h.pd_decouple, h.pd_stats = int(g["decouple"]), int(stats)
        num_f32, den_f32 = np.float32(0.0), np.float32(0.0)
        const = np.float32(d_over_d0 * dlr)
        for prm in self.params:
            t = _pd_tensor(prm, g, None if noise is None else noise.get(prm.tensor_id))
            num, den = ctypes.c_float(0.0), ctypes.c_float(0.0)
            _check(lib().ko_kprodigy_pass1_tensor(ctypes.byref(t), ctypes.byref(h), ctypes.byref(num),
                                                  ctypes.byref(den)))
            if stats:
                num_f32 = np.float32(num_f32 + np.float32(const * np.float32(num.value)))
                den_f32 = np.float32(den_f32 + np.float32(den.value))
        if should_update_d and lr > 0.0:
            if float(den_f32) > 0.0:
                global_num = d_numerator + float(num_f32)
                d_hat = g["d_coef"] * global_num / float(den_f32)
                if d == d0:
                    d = max(d, d_hat)
                d_max = max(d_max, d_hat)
                d = min(d_max, d * g["growth_rate"])
                g.update(d_numerator=global_num, d=d, d_max=d_max, d_hat=d_hat)
        # pass 2 takes the updated d (the denominator floor d*eps, and r*c/d) with the
        # dlr of the old d (kprodigy.py:366-386)
        h.pd_d = d
        for prm in self.params:
            prm.state["step"] += 1
            t = _pd_tensor(prm, g, None if noise is None else noise.get(prm.tensor_id))
            _check(lib().ko_kprodigy_pass2_tensor(ctypes.byref(t), ctypes.byref(h)))
        g["k"] = k + 1

    def global_mnorm(self) -> float:
        """msam.py:191-199 in the canonical order: each tensor's sum of squares
        (ko_momentum_sumsq), added in param order in fp32, fp32 sqrt."""
        sq = np.float32(0.0)
        for prm in self.params:
            t = _tensor(prm, self.group["momentum_dtype"])
            sq = np.float32(sq + np.float32(lib().ko_momentum_sumsq(ctypes.byref(t))))
        return float(np.sqrt(sq, dtype=np.float32))

    def tensor_factor(self, prm: OParam, sign: float) -> float:
        """MSAM norm="tensor" (msam.py:219-222): scale = (sign * rho) / (||m|| + eps)
        in fp32 as torch evaluates a python scalar over a tensor, reciprocal(norm + eps)
        * (sign * rho); ||m|| the fp32 square root of the tensor's sum of squares."""
        t = _tensor(prm, self.group["momentum_dtype"])
        s = np.float32(lib().ko_momentum_sumsq(ctypes.byref(t)))
        nrm = np.sqrt(s, dtype=np.float32)
        rec = np.float32(1.0) / np.float32(nrm + np.float32(self.meps))
        return float(np.float32(rec * np.float32(sign * self.rho)))

    def _msam_tensor_apply(self, sign: float, noise: dict[int, list] | None, step: int | None = None) -> None:
        h = _hyper(self.group, self.seed, self.t if step is None else step)
        stream = 0 if sign < 0 else 2
        for prm in self.params:
            if "m" not in prm.state:
                continue
            f = self.tensor_factor(prm, sign)
            t = _tensor(prm, self.group["momentum_dtype"], None if noise is None else noise.get(prm.tensor_id))
            lib().ko_msam_apply(ctypes.byref(t), ctypes.byref(h), f, math.inf, stream)

    def _msam_tensor_step(self, noise: dict[int, list] | None) -> None:
        """MSAM.step with norm="tensor" (msam.py:375-406): remove the previous climb
        with each tensor's own radius, the inner step, climb along the new momentum."""
        if self.has_e:
            self._msam_tensor_apply(-1.0, noise)
            self.has_e = False
        h = _hyper(self.group, self.seed, self.t)
        for prm in self.params:
            if prm.g is None:
                continue
            t = _tensor(prm, self.group["momentum_dtype"], None if noise is None else noise.get(prm.tensor_id))
            _check(lib().ko_adakaon_tensor(ctypes.byref(t), ctypes.byref(h)))
        if self.rho != 0.0 and any("m" in prm.state for prm in self.params):
            self._msam_tensor_apply(+1.0, noise)
            self.has_e = True

    def _msam_global_step(self, noise: dict[int, list] | None) -> None:
        """MSAM.step with norm="global" (msam.py:375-406): remove the previous climb
        (folded into the Adakaon step, factor -rho/(||m||+eps) with the cached norm,
        no bound), the inner step, then climb along the new momentum with its norm."""
        h = _hyper(self.group, self.seed, self.t)
        h.nk_remove = int(self.has_e)
        h.nk_k = -self.rho / (self.mnorm + self.meps)
        h.nk_bound_old = math.inf
        h.nk_climb = 0
        for prm in self.params:
            t = _tensor(prm, self.group["momentum_dtype"], None if noise is None else noise.get(prm.tensor_id))
            if prm.g is None:
                # no gradient this step: the param is not stepped, but MSAM removes the
                # climb from every param with a momentum (msam.py:155-167, 384-388)
                if h.nk_remove and "m" in prm.state:
                    lib().ko_msam_apply(ctypes.byref(t), ctypes.byref(h), h.nk_k, math.inf, 0)
                continue
            _check(lib().ko_adakaon_tensor(ctypes.byref(t), ctypes.byref(h)))
        self.has_e = False
        if self.rho != 0.0:
            own = self.global_mnorm()
            self.mnorm_log.append(own)
            self.mnorm = self.mnorm_feed.pop(0) if self.mnorm_feed else own
            if self.mnorm > 0.0:
                self.msam_apply(+1.0, noise)
                self.has_e = True

    def step(self, noise: dict[int, list] | None = None, fac_override: dict[int, np.ndarray] | None = None,
             ss_out: dict[int, np.ndarray] | None = None) -> None:
        """One step.  ``fac_override`` injects clip divisors per tensor id;
        ``ss_out`` (tensor id -> float32 [1]) receives the clip's sum of squares
        of the Adakaon / Nekaon / MSAM / AdaMuon / AdaPNM steps."""
        self.t += 1
        if self.opt == "kprodigy":
            self._kprodigy_step(noise)
            return
        if self.opt == "msam" and self.norm == "global":
            self._msam_global_step(noise)
            return
        if self.opt == "msam" and self.norm == "tensor":
            self._msam_tensor_step(noise)
            return
        h = _hyper(self.group, self.seed, self.t)
        md = self.group["momentum_dtype"]
        if self.opt in ("nekaon", "msam"):
            h.nk_remove = int(self.has_e)
            h.nk_bound_old = self.bound
            new_bound = abs(self.k) * self.group.get("clip_threshold", 1.0) * self.group["lr"]
            h.nk_climb = int(self.k != 0.0)
            h.nk_k = self.k
            h.nk_bound_new = new_bound
        for prm in self.params:
            if prm.g is None:
                # the reference skips a param without a gradient; MSAM still removes and
                # re-adds the climb on every param with a momentum (msam.py:384-403)
                if self.opt in ("nekaon", "msam") and "m" in prm.state:
                    t = _tensor(prm, md, None if noise is None else noise.get(prm.tensor_id))
                    if h.nk_remove:
                        lib().ko_msam_apply(ctypes.byref(t), ctypes.byref(h), h.nk_k, h.nk_bound_old, 0)
                    if h.nk_climb:
                        lib().ko_msam_apply(ctypes.byref(t), ctypes.byref(h), -h.nk_k, h.nk_bound_new, 2)
                continue
            if self.opt == "adapnm":
                t = _pnm_tensor(prm, md, self.t, None if noise is None else noise.get(prm.tensor_id))
                t.ss_out = _ptr(None if ss_out is None else ss_out.get(prm.tensor_id))
                _check(lib().ko_adapnm_tensor(ctypes.byref(t), ctypes.byref(h)))
                continue
            t = _tensor(prm, md, None if noise is None else noise.get(prm.tensor_id),
                        fac_override=None if fac_override is None else fac_override.get(prm.tensor_id),
                        ss_out=None if ss_out is None else ss_out.get(prm.tensor_id))
            if self.opt in ("adakaon", "nekaon", "msam"):
                _check(lib().ko_adakaon_tensor(ctypes.byref(t), ctypes.byref(h)))
            elif self.opt == "lion":
                _check(lib().ko_lion_tensor(ctypes.byref(t), ctypes.byref(h)))
            elif self.opt == "adamuon":
                _check(lib().ko_adamuon_tensor(ctypes.byref(t), ctypes.byref(h)))
            else:
                raise ValueError(self.opt)
        if self.opt in ("nekaon", "msam") and self.k != 0.0:
            self.has_e = True
            self.bound = h.nk_bound_new

    def msam_apply(self, sign: float, noise: dict[int, list] | None = None, step: int | None = None) -> None:
        """MSAM._apply(sign) with the frozen bound (eval(): sign=-1; train(): +1).

        ``step`` keys the SR noise (default: the current step count).  A caller
        that drives MSAM over another optimizer by hand sets ``rho``, ``norm``,
        ``meps`` (and ``mnorm`` from :meth:`global_mnorm`) on this object."""
        if self.norm == "tensor":
            self._msam_tensor_apply(sign, noise, step)
            return
        h = _hyper(self.group, self.seed, self.t if step is None else step)
        factor = sign * (-self.k)
        bound = self.bound
        if self.norm == "global":
            factor, bound = sign * self.rho / (self.mnorm + self.meps), math.inf
        stream = 0 if sign < 0 else 2
        for prm in self.params:
            t = _tensor(prm, self.group["momentum_dtype"], None if noise is None else noise.get(prm.tensor_id))
            lib().ko_msam_apply(ctypes.byref(t), ctypes.byref(h), factor, bound, stream)


def make_param(shape, p_dtype=BF16, g_dtype=BF16, tensor_id=0, *, p_values=None, g_values=None) -> OParam:
    shape = tuple(int(s) for s in shape)
    def conv(v, dt):
        v = np.ascontiguousarray(v, dtype=np.float32).reshape(shape)
        if dt == BF16:
            return f32_to_bf16(v).reshape(shape)
        return f32_to_f16(v).reshape(shape) if dt == F16 else v.copy()
    prm = OParam(p=conv(p_values, p_dtype), p_dtype=p_dtype, shape=shape, tensor_id=tensor_id,
                 g_dtype=g_dtype)
    if g_values is not None:
        prm.g = conv(g_values, g_dtype)
    return prm


def values(a: np.ndarray, dtype: int) -> np.ndarray:
    if dtype == BF16:
        return bf16_to_f32(a)
    return f16_to_f32(a) if dtype == F16 else a.astype(np.float32)


__all__ = [
    "BF16", "F16", "F32", "KoHyper", "KoTensor", "OParam", "OracleOptimizer", "TORCH_ORDER", "bf16_to_f32", "csum",
    "dequant", "f16_to_f32", "f32_to_bf16", "f32_to_f16", "fourbit_block_size", "gc_bf16", "init_state", "lerp", "lib", "make_param",
    "newton_schulz", "philox4x32_10", "quant_4bit", "quant_int8", "rows_per_wave", "sr_noise", "sr_round",
    "torch_inner_sum", "torch_order", "torch_outer_sum", "torch_sumsq", "values",
]
_ = math
