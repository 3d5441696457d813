"""ctypes binding of ``libkaon_amd.so`` (the C ABI declared in ``include/kaon_amd.h``).

The structures below mirror the header field for field.  The library is
loaded from this package directory only; when it is missing the import of the
optimizers fails with a RuntimeError -- there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libkaon_amd.so")

ABI_VERSION = 10

F32, BF16, F16 = 0, 1, 2
MOM_NONE, MOM_F32, MOM_BF16, MOM_INT8, MOM_4BIT = 0, 1, 2, 3, 4
MOM_CODE = {"none": MOM_NONE, "float32": MOM_F32, "bfloat16": MOM_BF16, "int8": MOM_INT8, "4bit": MOM_4BIT}
SR, RN, KAHAN = 0, 1, 2
BF16_METHOD = {"stochastic_rounding": SR, "none": RN, "kahan": KAHAN}
OPT_ADAKAON, OPT_LION, OPT_ADAMUON, OPT_ADAPNM, OPT_KPRODIGY = 0, 1, 2, 3, 4

F_GC, F_CAUTIOUS, F_WD, F_EPS, F_MOMENTUM, F_NK_REMOVE, F_NK_CLIMB, F_SRC_O = 1, 2, 4, 8, 16, 32, 64, 128
F_GC_WRITE = 4096
F_TORCH_ORDER = 8192
F_PD_BLOCKFAC = 16384
F_PNM, F_AMS, F_PD_COUPLED, F_PD_STATS = 256, 512, 1024, 2048

ROW_BUDGET = 20
ROW_CLASSES = 7
COLITEM = 2048
FLAT_ITEM = 16384
NS_TILE = 128
NS_XCDS = 8  # KAON_NS_XCDS: big Newton-Schulz tiles are laid out per XCD


class KaonTensor(ctypes.Structure):
    _fields_ = [
        ("g", ctypes.c_void_p), ("p", ctypes.c_void_p), ("m", ctypes.c_void_p),
        ("m_scale", ctypes.c_void_p), ("row", ctypes.c_void_p), ("col", ctypes.c_void_p),
        ("v", ctypes.c_void_p), ("shift", ctypes.c_void_p),
        ("m2", ctypes.c_void_p), ("m2_scale", ctypes.c_void_p), ("max_v", ctypes.c_void_p),
        ("pd_s", ctypes.c_void_p), ("pd_p0", ctypes.c_void_p), ("pd_ns", ctypes.c_int64),
        ("pd_slice", ctypes.c_int32), ("pd_p0_scalar", ctypes.c_int32), ("full_v", ctypes.c_int32),
        ("by_size", ctypes.c_int32),
        ("noise", ctypes.c_void_p * 3),
        ("R", ctypes.c_int64), ("C", ctypes.c_int64), ("n", ctypes.c_int64),
        ("ws_row", ctypes.c_int64), ("ws_col", ctypes.c_int64), ("ws_part", ctypes.c_int64),
        ("ws_blk", ctypes.c_int64), ("ws_scal", ctypes.c_int64), ("ws_aux", ctypes.c_int64),
        ("tensor_id", ctypes.c_int32), ("block4", ctypes.c_int32), ("factored", ctypes.c_int32),
        ("ngroups", ctypes.c_int32), ("sqrt_n", ctypes.c_float),
        ("vec_rows", ctypes.c_int32), ("vec_flat", ctypes.c_int32), ("ns_tr", ctypes.c_int32),
        ("m_pad", ctypes.c_int32), ("k_pad", ctypes.c_int32), ("fast_lanes", ctypes.c_int32),
        ("gc_write", ctypes.c_int32), ("fb_r", ctypes.c_int32), ("fb_c", ctypes.c_int32),
    ]


class KaonItem(ctypes.Structure):
    _fields_ = [("tensor", ctypes.c_int32), ("row0", ctypes.c_int32), ("nrows", ctypes.c_int32),
                ("kind", ctypes.c_int32)]


class KaonPlanInfo(ctypes.Structure):
    _fields_ = [("n_tensors", ctypes.c_int32), ("n_row_items", ctypes.c_int32),
                ("n_fin_items", ctypes.c_int32), ("n_flat_items", ctypes.c_int32),
                ("row_runs", ctypes.c_int32 * ROW_CLASSES), ("n_fast", ctypes.c_int32),
                ("n_elem_items", ctypes.c_int32), ("n_ns_sq", ctypes.c_int32), ("n_ns_rect", ctypes.c_int32),
                ("n_ns_sq_big", ctypes.c_int32), ("n_ns_rect_big", ctypes.c_int32), ("ws_words", ctypes.c_int64),
                ("n_long", ctypes.c_int32), ("n_long_fast", ctypes.c_int32), ("n_long_rest", ctypes.c_int32),
                ("reserved", ctypes.c_int32)]


class KaonPlanArgs(ctypes.Structure):
    _fields_ = [("opt", ctypes.c_int32), ("codec", ctypes.c_int32), ("p_dtype", ctypes.c_int32),
                ("g_dtype", ctypes.c_int32), ("bf16_method", ctypes.c_int32)]


class KaonLaunch(ctypes.Structure):
    _fields_ = [("descs", ctypes.c_void_p), ("row_items", ctypes.c_void_p), ("elem_items", ctypes.c_void_p),
                ("fin_items", ctypes.c_void_p), ("flat_items", ctypes.c_void_p),
                ("ns_sq_items", ctypes.c_void_p), ("ns_rect_items", ctypes.c_void_p),
                ("n_tensors", ctypes.c_int32), ("n_row_items", ctypes.c_int32),
                ("n_fin_items", ctypes.c_int32), ("n_flat_items", ctypes.c_int32),
                ("row_runs", ctypes.c_int32 * ROW_CLASSES), ("n_fast", ctypes.c_int32),
                ("n_elem_items", ctypes.c_int32), ("n_ns_sq", ctypes.c_int32), ("n_ns_rect", ctypes.c_int32),
                ("n_ns_sq_big", ctypes.c_int32), ("n_ns_rect_big", ctypes.c_int32), ("workspace", ctypes.c_void_p),
                ("ws_words", ctypes.c_int64), ("n_long", ctypes.c_int32), ("n_long_fast", ctypes.c_int32),
                ("n_long_rest", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class KaonHyper(ctypes.Structure):
    _fields_ = [
        ("lr", ctypes.c_float), ("w1", ctypes.c_float), ("w2", ctypes.c_float), ("eps1", ctypes.c_float),
        ("wdl", ctypes.c_float), ("clip", ctypes.c_float), ("b1", ctypes.c_float), ("b2", ctypes.c_float),
        ("a1", ctypes.c_float), ("a2", ctypes.c_float), ("nk_k", ctypes.c_float),
        ("nk_bound_old", ctypes.c_float), ("nk_bound_new", ctypes.c_float),
        ("pn_pos", ctypes.c_float), ("pn_neg", ctypes.c_float), ("pn_rnorm", ctypes.c_float),
        ("bc2", ctypes.c_float),
        ("pd_tg", ctypes.c_float), ("pd_vval", ctypes.c_float), ("pd_alpha_s", ctypes.c_float),
        ("pd_beta3", ctypes.c_float), ("pd_d", ctypes.c_float), ("pd_dn", ctypes.c_float),
        ("pd_floor", ctypes.c_float),
        ("pd_cap", ctypes.c_float), ("pd_dlr", ctypes.c_float), ("pd_wdl", ctypes.c_float),
        ("flags", ctypes.c_int32), ("p_dtype", ctypes.c_int32), ("g_dtype", ctypes.c_int32),
        ("codec", ctypes.c_int32), ("bf16_method", ctypes.c_int32), ("ns_steps", ctypes.c_int32),
        ("step", ctypes.c_uint32), ("seed", ctypes.c_uint64),
    ]


assert ctypes.sizeof(KaonTensor) == 280, ctypes.sizeof(KaonTensor)
assert ctypes.sizeof(KaonItem) == 16
assert ctypes.sizeof(KaonHyper) == 144, ctypes.sizeof(KaonHyper)

# entry points: name -> (argtypes, restype)
_VP, _I32, _I64, _U32, _U64, _F = (ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32,
                                   ctypes.c_uint64, ctypes.c_float)
SIGNATURES = {
    "kaon_abi_version": ([], ctypes.c_int),
    "kaon_last_error": ([], ctypes.c_char_p),
    "kaon_plan": ([ctypes.POINTER(KaonPlanArgs), _VP, _I32, _VP, _VP, _VP, _VP, _VP, _VP,
                   ctypes.POINTER(KaonPlanInfo)], ctypes.c_int),
    "kaon_adakaon_step": ([ctypes.POINTER(KaonLaunch), ctypes.POINTER(KaonHyper), _VP], ctypes.c_int),
    "kaon_gc_writeback": ([ctypes.POINTER(KaonLaunch), ctypes.POINTER(KaonHyper), _VP], ctypes.c_int),
    "kaon_adakaon_step_noalloc": ([ctypes.POINTER(KaonLaunch), ctypes.POINTER(KaonHyper), _VP], ctypes.c_int),
    "kaon_lion_step": ([ctypes.POINTER(KaonLaunch), ctypes.POINTER(KaonHyper), _VP], ctypes.c_int),
    "kaon_adamuon_step": ([ctypes.POINTER(KaonLaunch), ctypes.POINTER(KaonHyper), _VP], ctypes.c_int),
    "kaon_adapnm_step": ([ctypes.POINTER(KaonLaunch), ctypes.POINTER(KaonHyper), _VP], ctypes.c_int),
    "kaon_kprodigy_pass1": ([ctypes.POINTER(KaonLaunch), ctypes.POINTER(KaonHyper), _VP], ctypes.c_int),
    "kaon_kprodigy_pass2": ([ctypes.POINTER(KaonLaunch), ctypes.POINTER(KaonHyper), _VP], ctypes.c_int),
    "kaon_adakaon_phases": ([ctypes.POINTER(KaonLaunch), ctypes.POINTER(KaonHyper), _U32, _VP], ctypes.c_int),
    "kaon_lion_phases": ([ctypes.POINTER(KaonLaunch), ctypes.POINTER(KaonHyper), _U32, _VP], ctypes.c_int),
    "kaon_adamuon_phases": ([ctypes.POINTER(KaonLaunch), ctypes.POINTER(KaonHyper), _U32, _VP], ctypes.c_int),
    "kaon_adapnm_phases": ([ctypes.POINTER(KaonLaunch), ctypes.POINTER(KaonHyper), _U32, _VP], ctypes.c_int),
    "kaon_msam_apply": ([ctypes.POINTER(KaonLaunch), ctypes.POINTER(KaonHyper), _F, _F, _U32, _VP], ctypes.c_int),
    "kaon_msam_apply_tensor": ([ctypes.POINTER(KaonLaunch), ctypes.POINTER(KaonHyper), _F, _F, _U32, _VP],
                               ctypes.c_int),
    "kaon_momentum_sumsq": ([ctypes.POINTER(KaonLaunch), ctypes.POINTER(KaonHyper), _VP], ctypes.c_int),
    "kaon_quant_int8": ([_VP, _I64, _I64, _VP, _VP, _VP], ctypes.c_int),
    "kaon_quant_4bit": ([_VP, _I64, _I32, _VP, _VP, _VP], ctypes.c_int),
    "kaon_dequant": ([_I32, _VP, _VP, _I64, _I64, _I32, _VP, _VP], ctypes.c_int),
    "kaon_sr_round": ([_VP, _VP, _I64, _VP, _VP], ctypes.c_int),
    "kaon_sr_noise": ([_VP, _I64, _U64, _U32, _U32, _U32, _VP], ctypes.c_int),
    "kaon_copy": ([_VP, _VP, _I64, _VP], ctypes.c_int),
    "kaon_apply_ceiling": ([_VP, _VP, _VP, _I64, _VP], ctypes.c_int),
}

_handle: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The HIP library; raises RuntimeError when it has not been built."""
    global _handle
    if _handle is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"kaon_amd: HIP library not built ({LIB_PATH}); run "
                "`python -c 'import __graft_entry__ as g; g.build()'` or `make -C k-optimizers_amd/csrc`")
        h = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(h, name)
            fn.argtypes = args
            fn.restype = res
        if h.kaon_abi_version() != ABI_VERSION:
            raise RuntimeError(f"kaon_amd: ABI version {h.kaon_abi_version()} != {ABI_VERSION}")
        _handle = h
    return _handle


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().kaon_last_error()
        raise RuntimeError(f"{what} failed ({rc}): {msg.decode() if msg else ''}")
