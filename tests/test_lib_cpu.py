"""CPU checks of the C-ABI library: exports, struct layout, host-side planning.

No GPU is touched: kaon_plan is host code, and symbol / layout checks only load
the shared object.
"""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "kaon_amd.h")


def _lib():
    from kaon_amd import _lib

    return _lib


def test_library_exports_every_declared_symbol():
    src = open(HEADER).read()
    names = set(re.findall(r"^\s*(?:int|const char\*)\s+(kaon_\w+)\s*\(", src, re.M))
    assert {"kaon_plan", "kaon_adakaon_step", "kaon_lion_step", "kaon_msam_apply"} <= names
    h = ctypes.CDLL(_lib().LIB_PATH)
    missing = [n for n in sorted(names) if not hasattr(h, n)]
    assert not missing, missing
    assert set(_lib().SIGNATURES) >= names
    assert _lib().lib().kaon_abi_version() == _lib().ABI_VERSION


def test_struct_layout_matches_c_compiler(tmp_path):
    L = _lib()
    structs = {"KaonTensor": L.KaonTensor, "KaonItem": L.KaonItem, "KaonPlanInfo": L.KaonPlanInfo,
               "KaonLaunch": L.KaonLaunch, "KaonHyper": L.KaonHyper}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "kaon_amd.h"', "int main(void){"]
    for sname, cls in structs.items():
        lines.append(f'printf("{sname} size %zu\\n", sizeof({sname}));')
        for fname, _t in cls._fields_:
            lines.append(f'printf("{sname} {fname} %zu\\n", offsetof({sname}, {fname}));')
    lines.append("return 0;}")
    c = tmp_path / "layout.c"
    c.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.dirname(HEADER), str(c), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = {}
    for ln in out:
        if ln:
            s, f, v = ln.split()
            got[(s, f)] = int(v)
    for sname, cls in structs.items():
        assert got[(sname, "size")] == ctypes.sizeof(cls), sname
        for fname, _t in cls._fields_:
            assert got[(sname, fname)] == getattr(cls, fname).offset, (sname, fname)


def _plan(shapes, opt=0, codec=3, block=128, g_dtype=1):
    L = _lib()
    n = len(shapes)
    descs = (L.KaonTensor * n)()
    for i, s in enumerate(shapes):
        d = descs[i]
        numel = int(np.prod(s))
        if len(s) >= 2:
            d.R, d.C, d.factored = s[0], numel // s[0], 1
        else:
            d.R, d.C, d.factored = 1, numel, 0
        d.block4 = min(block, numel) if numel else 1
        d.tensor_id = i
        d.g = d.p = d.m = d.m_scale = 0x1000 * (i + 1)
    info = L.KaonPlanInfo()
    args = L.KaonPlanArgs(opt, codec, 1, g_dtype, 0)
    rc = L.lib().kaon_plan(ctypes.byref(args), descs, n, None, None, None, None, None, None, ctypes.byref(info))
    if rc:
        return rc, None, None, None, None, None
    rows = (L.KaonItem * max(info.n_row_items, 1))()
    elems = (L.KaonItem * max(info.n_elem_items, 1))()
    fins = (L.KaonItem * max(info.n_fin_items, 1))()
    flats = (L.KaonItem * max(info.n_flat_items, 1))()
    assert L.lib().kaon_plan(ctypes.byref(args), descs, n, rows, elems, fins, flats, None, None,
                             ctypes.byref(info)) == 0
    # phase-5/6 items: specialized-kernel ones first; every row of every
    # tensor exactly once; the generic kernel's are slices of 4 wave groups
    covered = {i: np.zeros(descs[i].R, np.int32) for i in range(n) if descs[i].R * descs[i].C > 0}
    for k in range(info.n_elem_items):
        it = elems[k]
        d = descs[it.tensor]
        fast = (g_dtype == 1 and d.factored == 1 and d.vec_rows == 1 and d.C % 8 == 0 and d.R * d.C <= 1 << 31
                and (codec != 4 or (d.block4 % 8 == 0 and 64 % (d.block4 // 8) == 0)))
        assert (k < info.n_fast) == fast, (k, d.R, d.C)
        covered[it.tensor][it.row0:it.row0 + it.nrows] += 1
        if fast:
            gl = d.block4 // 8 if codec == 4 else 1
            assert d.fast_lanes == _fast_lanes(d.C, gl), (d.C, d.fast_lanes)
            per = 64 // d.fast_lanes
            assert it.kind % per == 0 and it.kind >= _rows_per_wave(d.C) > it.kind - per
            assert it.row0 % (4 * it.kind) == 0 and 0 < it.nrows <= 4 * it.kind
        else:
            assert it.kind == _rows_per_wave(d.C) if d.factored else it.nrows == 1
            assert it.row0 % (4 * it.kind) == 0 and 0 < it.nrows <= 4 * it.kind
    assert all((v == 1).all() for v in covered.values())
    return 0, descs, info, rows, fins, flats


def _rows_per_wave(C):
    return max(1, 20 // _cpl(C))


def _fast_lanes(C, gl):
    """Lanes per row of the specialized phase-5/6 kernel: the power of two in
    [max(8, gl), 64] with the fewest idle lanes over a row's C/8 chunks, ties
    to the larger (checked by brute force over the candidates)."""
    nfull = C // 8
    use = {L: nfull / (L * -(-nfull // L)) for L in (64, 32, 16, 8) if L >= gl}
    best = max(use.values())
    return max(L for L, u in use.items() if u >= best - 1e-12)


def _cpl(C):
    return max(1, -(-(-(-C // 8)) // 64))


@pytest.mark.parametrize("g_dtype", [0, 1])
def test_plan_covers_every_row_and_element_once(g_dtype):
    import oracle as O

    shapes = [(1280, 1280, 3, 3), (640, 640, 3, 3), (5120, 1280), (1280, 2048), (77, 33), (1280,), (5,), (3, 5, 7),
              (9, 1), (2, 16384), (50, 12288), (7, 2880)]
    rc, descs, info, rows, fins, flats = _plan(shapes, codec=4, block=64, g_dtype=g_dtype)
    assert rc == 0
    L = _lib()
    assert sum(info.row_runs) == info.n_row_items
    # slices: every row of every tensor exactly once, classes ascending, the
    # rows-per-wave of the oracle's column-sum order
    seen = {i: np.zeros(descs[i].R, np.int32) for i in range(len(shapes))}
    off = 0
    for cls in range(L.ROW_CLASSES):
        for k in range(info.row_runs[cls]):
            it = rows[off + k]
            d = descs[it.tensor]
            seen[it.tensor][it.row0:it.row0 + it.nrows] += 1
            # runs of KAON_RUN = 4 slices of 4 wave groups of RW rows
            assert it.kind == O.rows_per_wave(d.C)
            assert it.nrows <= 16 * it.kind and it.row0 % (16 * it.kind) == 0
            cpl = _cpl(d.C)
            prefetch = g_dtype == 1 and d.factored and d.vec_rows and d.C % 8 == 0 and cpl <= 24
            if not d.factored:
                assert cls == 6
            elif prefetch:
                assert cls == (0 if cpl <= 4 else 1 if cpl <= 10 else 2)
            elif cls < 6:
                assert 3 <= cls and cpl <= (4, 10, 24)[cls - 3] and (cls < 5 or g_dtype == 1)
            else:
                assert cpl > 24 or (cpl > 10 and g_dtype == 0)
        off += info.row_runs[cls]
    assert all((v == 1).all() for v in seen.values())
    # flat items: every element exactly once, 8-aligned starts
    cover = {i: 0 for i in range(len(shapes))}
    for k in range(info.n_flat_items):
        it = flats[k]
        assert it.row0 % 8 == 0 and it.nrows <= L.FLAT_ITEM
        cover[it.tensor] += it.nrows
    assert all(cover[i] == descs[i].n for i in range(len(shapes)))
    # fin items: columns of factored tensors once + one row-stat item each
    for i in range(len(shapes)):
        d = descs[i]
        cols = sum(fins[k].nrows for k in range(info.n_fin_items) if fins[k].tensor == i and fins[k].kind == 0)
        rstat = sum(1 for k in range(info.n_fin_items) if fins[k].tensor == i and fins[k].kind == 1)
        assert (cols, rstat) == ((d.C, 1) if d.factored else (0, 0))
    # workspace regions are disjoint and in bounds
    spans = []
    for i in range(len(shapes)):
        d = descs[i]
        nb = -(-d.n // d.block4)
        spans.append((d.ws_row, d.ws_row + 5 * d.R))
        if d.factored:
            spans.append((d.ws_col, d.ws_col + d.C))
            spans.append((d.ws_part, d.ws_part + 2 * d.ngroups * d.C))  # G^2 and the clip's G^2 / row
        spans.append((d.ws_blk, d.ws_blk + 2 * nb))
        spans.append((d.ws_scal, d.ws_scal + 5 + (-(-d.C // 2048) if d.factored else 1)))
        assert d.ngroups == -(-d.R // (16 * O.rows_per_wave(d.C)))
        assert d.sqrt_n == np.float32(np.sqrt(float(max(d.n, 1))))
    spans.sort()
    for (a0, a1), (b0, _b1) in zip(spans, spans[1:]):
        assert a1 <= b0
    assert spans[-1][1] <= info.ws_words
    # vector flags: rows need C % 8 == 0 (or a single row)
    for i, s in enumerate(shapes):
        assert descs[i].vec_rows == (1 if (descs[i].C % 8 == 0 or descs[i].R == 1) else 0)


def test_plan_takes_rows_of_any_length():
    """Rows longer than any register class (SDXL up-block convs [640,1920,3,3] and
    [1280,2560,3,3], rows of 17280 and 23040; a 28672-input linear) are planned as
    streamed rows (class 6) with one run per 4 slices of 4 rows."""
    shapes = [(640, 1920, 3, 3), (1280, 2560, 3, 3), (4096, 28672), (4, 16385)]
    rc, descs, info, rows, _fins, _flats = _plan(shapes)
    assert rc == 0
    assert info.row_runs[6] == sum(-(-s[0] // 16) for s in shapes)
    for i in range(len(shapes)):
        assert descs[i].ngroups == -(-descs[i].R // 16)


def test_constructor_validation_mirrors_reference():
    from kaon_amd import Adakaon, Lion, Nekaon

    p = [torch.nn.Parameter(torch.zeros(4, 4))]
    for bad in (dict(betas=(1.0, 0.9)), dict(betas=(0.9, -0.1)), dict(lr=-1.0), dict(clip_threshold=0.0),
                dict(momentum_dtype="int4"), dict(bf16_method="round"), dict(foreach_batch_cutoff=0)):
        with pytest.raises(ValueError):
            Adakaon(p, **bad)
    with pytest.raises(ValueError):
        Lion(p, weight_decay=-0.1)
    with pytest.raises(ValueError):
        Nekaon(p, k=-1.0)
    with pytest.raises(ValueError):
        Nekaon(p, betas=(0.0, 0.999))
    with pytest.raises(TypeError):
        Nekaon([{"params": p}], low_vram_above=10)


def test_cpu_params_fail_loudly():
    """There is no CPU fallback: a step on CPU tensors raises."""
    from kaon_amd import Adakaon

    p = torch.nn.Parameter(torch.zeros(4, 4))
    p.grad = torch.ones(4, 4)
    opt = Adakaon([p])
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        opt.step()


def test_state_layout_matches_reference_at_init():
    """_init_state layouts (adakaon.py:318-335, _momentum_codec.py:293-361) on CPU tensors."""
    from kaon_amd import Adakaon, Lion
    from kaon_amd._base import init_momentum_state

    conv = torch.nn.Parameter(torch.zeros(8, 4, 3, 3, dtype=torch.bfloat16))
    conv.grad = torch.zeros_like(conv)
    vec = torch.nn.Parameter(torch.zeros(10))
    vec.grad = torch.zeros_like(vec)
    opt = Adakaon([conv, vec], momentum_dtype="int8", bf16_method="kahan")
    st, sv = {}, {}
    opt._init_state(conv, st, opt.param_groups[0])
    opt._init_state(vec, sv, opt.param_groups[0])
    assert st["row"].shape == (8,) and st["col"].shape == (36,)
    assert st["m"].dtype == torch.int8 and st["m"].shape == conv.shape
    assert st["m_scale"].shape == (8, 1, 1, 1) and st["shift"].dtype == torch.bfloat16
    assert sv["v"].shape == (10,) and sv["m_scale"].shape == () and "shift" not in sv
    s4 = {}
    init_momentum_state(s4, vec.grad, dict(momentum_dtype="4bit", momentum_4bit_block=4))
    assert s4["m"].tolist() == [0x88] * 5 and s4["m_scale"].shape == (3,) and s4["m_block"] == 4
    lion = Lion([vec], momentum_dtype="bfloat16")
    sl = {}
    lion._init_state(vec, sl, lion.param_groups[0])
    assert sl["m"].dtype == torch.bfloat16 and set(sl) == {"m"}


def test_adamuon_plan_pads_and_tiles_newton_schulz():
    """AdaMuon plans: m_pad/k_pad round min/max(R, C) up to the GEMM tile (twice
    KAON_NS_TILE when m is at least 4 tiles and the padding to the big tile grows
    m^2 by at most 1.5x), the transposed flag marks R > C, every tile of the padded
    products is listed once (big symmetric products: row <= column only, big
    items first), and the Newton-Schulz blocks do not overlap other workspace."""
    L = _lib()
    shapes = [(1280, 1280, 3, 3), (5120, 1280), (77, 33), (320, 2880), (20, 12), (640, 640), (512, 2000),
              (1024, 5760)]
    n = len(shapes)
    descs = (L.KaonTensor * n)()
    for i, s in enumerate(shapes):
        d = descs[i]
        numel = int(np.prod(s))
        d.R, d.C, d.factored, d.tensor_id = s[0], numel // s[0], 1, i
        d.g = d.p = d.m = d.m_scale = 0x1000 * (i + 1)
    info = L.KaonPlanInfo()
    args = L.KaonPlanArgs(L.OPT_ADAMUON, L.MOM_INT8, L.BF16, L.BF16, L.SR)
    assert L.lib().kaon_plan(ctypes.byref(args), descs, n, None, None, None, None, None, None, ctypes.byref(info)) == 0
    sq = (L.KaonItem * info.n_ns_sq)()
    rect = (L.KaonItem * info.n_ns_rect)()
    assert L.lib().kaon_plan(ctypes.byref(args), descs, n, None, None, None, None, sq, rect, ctypes.byref(info)) == 0
    spans = []
    nbig_sq = nbig_rect = 0
    for i, s in enumerate(shapes):
        d = descs[i]
        m, k = min(d.R, d.C), max(d.R, d.C)
        m128 = -(-m // L.NS_TILE) * L.NS_TILE
        m256 = -(-m // (2 * L.NS_TILE)) * 2 * L.NS_TILE
        big = m128 >= 4 * L.NS_TILE and 2 * m256 * m256 <= 3 * m128 * m128
        assert big == (m in (1280, 512, 1024, 640)), (s, big)
        t = 2 * L.NS_TILE if big else L.NS_TILE
        assert d.ns_tr == (1 if d.R > d.C else 0)
        assert d.m_pad == -(-m // t) * t and d.k_pad == -(-k // t) * t
        got_sq = sorted((it.row0, it.nrows, it.kind) for it in sq if it.tensor == i)
        got_rect = sorted((it.row0, it.nrows, it.kind) for it in rect if it.tensor == i)
        tm, tk = d.m_pad // t, d.k_pad // t
        assert got_sq == [(a, b, int(big)) for a in range(tm) for b in range(tm) if not big or a <= b]
        assert got_rect == [(a, b, int(big)) for a in range(tm) for b in range(tk)]
        nbig_sq += len(got_sq) if big else 0
        nbig_rect += len(got_rect) if big else 0
        words = ((d.R * d.C + 1) // 2 + 3) // 4 * 4 + 2 * ((d.m_pad * d.k_pad // 2 + 3) // 4 * 4) \
            + 2 * ((d.m_pad * d.m_pad // 2 + 3) // 4 * 4)
        spans += [(d.ws_row, d.ws_row + 5 * d.R), (d.ws_col, d.ws_col + d.C),
                  (d.ws_part, d.ws_part + 2 * d.ngroups * d.C), (d.ws_scal, d.ws_scal + 5 + -(-d.C // 2048)),
                  (d.ws_aux, d.ws_aux + words)]
    spans.sort()
    for (a0, a1), (b0, _b1) in zip(spans, spans[1:]):
        assert a1 <= b0
    assert spans[-1][1] <= info.ws_words
    # the keep-count / apply slices of tensors with C % 8 == 0 (bf16, SR) go to the
    # specialized kernel and lead the list
    elems = (L.KaonItem * info.n_elem_items)()
    assert L.lib().kaon_plan(ctypes.byref(args), descs, n, None, elems, None, None, sq, rect,
                             ctypes.byref(info)) == 0
    assert info.n_fast > 0
    for j in range(info.n_elem_items):
        assert (j < info.n_fast) == (descs[elems[j].tensor].C % 8 == 0), (j, descs[elems[j].tensor].C)
    # big-tile items lead both lists, laid out per XCD: item 8 i + x is XCD x's
    # i-th tile, and a shorter XCD list ends in idle items (tensor -1)
    for items, nbig, nreal, sqk in ((sq, info.n_ns_sq_big, nbig_sq, True),
                                    (rect, info.n_ns_rect_big, nbig_rect, False)):
        X = L.NS_XCDS
        assert nbig % X == 0 and nbig >= nreal
        assert sum(items[j].tensor >= 0 for j in range(nbig)) == nreal
        assert all(items[j].kind == (j < nbig) for j in range(len(items)))
        assert all(items[j].tensor >= 0 for j in range(nbig, len(items)))
        loads = []
        for x in range(X):
            lst = [items[j] for j in range(x, nbig, X)]
            real = [it.tensor >= 0 for it in lst]
            assert real == sorted(real, reverse=True)  # idle items only at the end
            loads.append(sum((descs[it.tensor].k_pad + descs[it.tensor].m_pad) if sqk else descs[it.tensor].m_pad
                             for it in lst if it.tensor >= 0))
        # pieces are at most 1/64 of the work: no XCD gets much more than its share
        assert max(loads) <= sum(loads) / X * 1.2 + 1, loads


def test_adamuon_plan_rejects_1d():
    L = _lib()
    descs = (L.KaonTensor * 1)()
    descs[0].R, descs[0].C, descs[0].factored = 1, 40, 0
    info = L.KaonPlanInfo()
    args = L.KaonPlanArgs(L.OPT_ADAMUON, L.MOM_BF16, L.BF16, L.BF16, L.SR)
    assert L.lib().kaon_plan(ctypes.byref(args), descs, 1, None, None, None, None, None, None, ctypes.byref(info)) != 0
    assert "1-D" in L.lib().kaon_last_error().decode()


def test_adamuon_constructor_validation_mirrors_reference():
    from kaon_amd import AdaMuon

    p = [torch.nn.Parameter(torch.zeros(4, 4))]
    for bad in (dict(ns_steps=0), dict(betas=(1.0, 0.9)), dict(lr=-1.0), dict(clip_threshold=0.0),
                dict(momentum_dtype="fp8")):
        with pytest.raises(ValueError):
            AdaMuon(p, **bad)
    opt = AdaMuon(p)
    g = opt.param_groups[0]
    assert (g["lr"], g["betas"], g["ns_steps"], g["momentum_dtype"], g["gradient_centralization"]) == \
        (2e-2, (0.95, 0.999), 2, "bfloat16", False)


def test_fast_lanes_fill_every_lane_on_sdxl_rows():
    """Lanes per row of the phase-5/6 specialized kernel for the SDXL row
    lengths: every chunk round of these rows is full (C/8 = L * rounds)."""
    want = {1280: 32, 640: 16, 2048: 64, 5120: 64, 11520: 32, 5760: 16, 2880: 8, 320: 8}
    shapes = [(64, C) for C in want]
    rc, descs, info, _, _, _ = _plan(shapes, codec=3)
    assert rc == 0
    for i, C in enumerate(want):
        assert descs[i].fast_lanes == want[C], (C, descs[i].fast_lanes)
        assert (C // 8) % want[C] == 0
    # 4-bit blocks of 128 (16 chunks) keep at least 16 lanes per row
    rc, descs, info, _, _, _ = _plan([(64, 2880), (64, 1280)], codec=4, block=128)
    assert rc == 0
    assert descs[0].fast_lanes == 64 or descs[0].C % 128 != 0
    assert descs[1].fast_lanes == 32


def test_state_that_does_not_match_the_codec_is_refused():
    """State created for another momentum_dtype / betas, or for another shape, raises
    ValueError before anything is planned (the kernels would otherwise write past the
    buffer or read a missing one)."""
    from kaon_amd import _engine as E
    from kaon_amd import _lib as L

    p = torch.zeros(6, 10, dtype=torch.bfloat16)
    base = dict(p=p, g=p, R=6, C=10, factored=True, tensor_id=0, row=torch.zeros(6), col=torch.zeros(10))
    int8 = dict(base, m=torch.zeros(6, 10, dtype=torch.int8), m_scale=torch.ones(6, 1))
    E._check_state(int8, L.MOM_INT8, 0)                       # matches
    with pytest.raises(ValueError, match="dtype torch.int8"):  # momentum_dtype int8 -> bfloat16
        E._check_state(int8, L.MOM_BF16, 0)
    with pytest.raises(ValueError, match="'m' is missing"):   # betas[0] 0 -> 0.9
        E._check_state(dict(base), L.MOM_INT8, 0)
    four = dict(base, m=torch.full((30,), 0x88, dtype=torch.uint8), m_scale=torch.ones(1), block4=60)
    E._check_state(four, L.MOM_4BIT, 0)
    with pytest.raises(ValueError, match="'m_scale' has 1 elements"):  # block size changed to 16
        E._check_state(dict(four, block4=16), L.MOM_4BIT, 0)
    with pytest.raises(ValueError, match="'col' has 9 elements"):      # state of another shape
        E._check_state(dict(int8, col=torch.zeros(9)), L.MOM_INT8, 0)
    E._check_state(dict(base), L.MOM_NONE, 0)                 # beta1 = 0: no momentum needed


def test_plan_refuses_a_missing_momentum_buffer():
    L = _lib()
    descs = (L.KaonTensor * 1)()
    d = descs[0]
    d.R, d.C, d.factored, d.block4 = 8, 16, 1, 128
    d.g = d.p = 0x1000
    info = L.KaonPlanInfo()
    for codec in (1, 2, 3, 4):
        d.m, d.m_scale = None, None
        args = L.KaonPlanArgs(0, codec, 1, 1, 0)
        assert L.lib().kaon_plan(ctypes.byref(args), descs, 1, None, None, None, None, None, None,
                                 ctypes.byref(info)) != 0
        assert b"momentum" in L.lib().kaon_last_error()
    args = L.KaonPlanArgs(0, 0, 1, 1, 0)
    assert L.lib().kaon_plan(ctypes.byref(args), descs, 1, None, None, None, None, None, None,
                             ctypes.byref(info)) == 0


def test_plan_limits_for_tensors_of_2_to_the_31_elements_and_more():
    """Up to 2^32 - 1 elements: 2-D tensors of Adakaon and Lion plans are planned on
    the generic phase-5/6 kernel (the specialized one addresses bf16 by 32-bit byte
    offsets) with flat items whose element offsets pass 2^31; 1-D tensors, other
    optimizers and 2^32 elements are refused with a message."""
    L = _lib()
    big = (131073, 16384)  # 2^31 + 2^14 elements
    for opt in (0, 1):
        rc, descs, info, _rows, _fins, flats = _plan([big], opt=opt)
        assert rc == 0
        assert info.n_fast == 0
        offs = sorted((flats[k].row0 & 0xFFFFFFFF) for k in range(info.n_flat_items))
        assert offs[0] == 0 and offs[-1] == (descs[0].R * descs[0].C - 1) // 16384 * 16384
        assert all(b - a == 16384 for a, b in zip(offs, offs[1:]))
    for opt in (2, 3, 4):  # AdaMuon, AdaPNM, KProdigy
        assert _plan([big], opt=opt)[0] != 0
        assert b"2^31" in L.lib().kaon_last_error()
    assert _plan([(1 << 31,)])[0] != 0  # 1-D
    assert b"2^31" in L.lib().kaon_last_error()
    assert _plan([(1 << 16, 1 << 16)])[0] != 0  # 2^32
    assert b"2^32" in L.lib().kaon_last_error()


def check_noalloc_refuses_oversized_plans():
    """kaon_adakaon_step_noalloc checks the launch's own workspace size (KaonLaunch.ws_words,
    copied from the plan): a real plan larger than the static device array, or a launch
    that carries no size, is refused before anything touches a device."""
    L = _lib()
    descs = (L.KaonTensor * 2)()
    for i, (R, C) in enumerate(((262144, 2880), (640, 2880))):
        d = descs[i]
        d.R, d.C, d.factored, d.block4, d.tensor_id = R, C, 1, 128, i
        d.g = d.p = d.m = d.m_scale = 0x1000 * (i + 1)
    info = L.KaonPlanInfo()
    args = L.KaonPlanArgs(L.OPT_ADAKAON, L.MOM_INT8, L.BF16, L.BF16, L.SR)
    assert L.lib().kaon_plan(ctypes.byref(args), descs, 2, None, None, None, None, None, None,
                             ctypes.byref(info)) == 0
    cap = (32 * 1024 * 1024) // 4
    assert info.ws_words > cap
    fn = L.lib().kaon_adakaon_step_noalloc
    la, hp = L.KaonLaunch(), L.KaonHyper()
    la.n_tensors, la.n_row_items, la.ws_words = 2, info.n_row_items, info.ws_words
    assert fn(ctypes.byref(la), ctypes.byref(hp), None) != 0
    assert b"static workspace" in L.lib().kaon_last_error()
    la.ws_words = 0
    assert fn(ctypes.byref(la), ctypes.byref(hp), None) != 0
    assert b"no workspace size" in L.lib().kaon_last_error()


def test_noalloc_refuses_oversized_plans_before_any_launch():
    check_noalloc_refuses_oversized_plans()


def test_other_optimizers_refuse_torch_order():
    """The torch-order sums (KAON_F_TORCH_ORDER) are built for the Adakaon (Nekaon, MSAM)
    and Lion steps; the entry points of the other optimizers refuse the flag on the host,
    before any launch, rather than ignore it."""
    L = _lib()
    la, hp = L.KaonLaunch(), L.KaonHyper()
    la.n_tensors, la.n_row_items = 1, 1
    la.descs = la.workspace = 0x1000  # never dereferenced: the flag is refused first
    hp.flags = L.F_TORCH_ORDER
    hp.p_dtype = hp.g_dtype = L.BF16
    hp.codec = L.MOM_INT8
    for fn in ("kaon_adamuon_step", "kaon_adapnm_step", "kaon_kprodigy_pass1", "kaon_kprodigy_pass2"):
        assert getattr(L.lib(), fn)(ctypes.byref(la), ctypes.byref(hp), None) != 0, fn
        assert b"torch-order" in L.lib().kaon_last_error(), fn


def test_reduction_order_knob():
    from kaon_amd import Adakaon, Lion, Nekaon

    p = torch.nn.Parameter(torch.zeros(4, 4))
    assert Adakaon([p]).reduction_order == "canonical"
    assert Lion([p], reduction_order="torch").reduction_order == "torch"
    assert Nekaon([p], reduction_order="torch").inner.reduction_order == "torch"
    with pytest.raises(ValueError):
        Adakaon([p], reduction_order="cuda")


def test_plan_orders_tensors_longest_first():
    """kaon_plan's by_size: a permutation of the tensors by decreasing numel (stable), the
    order the per-tensor clip-norm workgroups take them in."""
    rc, descs, info, _rows, _fins, _flats = _plan([[64, 40], [1280], [640, 320, 3, 3], [64, 40], [7, 9], [40000]])
    assert rc == 0
    order = [descs[k].by_size for k in range(6)]
    assert sorted(order) == list(range(6))
    sizes = [descs[i].n for i in order]
    assert sizes == sorted(sizes, reverse=True)
    assert order.index(0) < order.index(3)  # equal sizes keep param order


def _plan_elems(shapes, opt=0):
    L = _lib()
    n = len(shapes)
    descs = (L.KaonTensor * n)()
    for i, s in enumerate(shapes):
        d = descs[i]
        numel = int(np.prod(s))
        d.R, d.C, d.factored = (s[0], numel // s[0], 1) if len(s) >= 2 else (1, numel, 0)
        d.block4 = 128
        d.tensor_id = i
        d.g = d.p = d.m = d.m_scale = 0x1000 * (i + 1)
    info = L.KaonPlanInfo()
    args = L.KaonPlanArgs(opt, 3, 1, 1, 0)
    assert L.lib().kaon_plan(ctypes.byref(args), descs, n, None, None, None, None, None, None, ctypes.byref(info)) == 0
    elems = (L.KaonItem * max(info.n_elem_items, 1))()
    assert L.lib().kaon_plan(ctypes.byref(args), descs, n, None, elems, None, None, None, None,
                             ctypes.byref(info)) == 0
    return descs, info, elems


def test_plan_marks_the_long_clip_chains():
    """The torch-order step's long-chain split (KaonPlanInfo.n_long*): the tensors of at
    least half the largest numel, a prefix of by_size, and their phase-5/6 items the
    leading ones of the specialized and of the generic items."""
    shapes = [[5120, 1280], [1280, 1280, 3, 3], [1280], [640, 11520], [1280, 11520], [8000000], [320, 2880]]
    descs, info, elems = _plan_elems(shapes)
    ns = [int(np.prod(s)) for s in shapes]
    thr = (max(ns) + 1) // 2
    long_t = {i for i, v in enumerate(ns) if v >= thr}
    assert info.n_long == len(long_t) == 4  # both 14.7M, the 7.37M conv, the 8M vector
    ranks = [descs[k].by_size for k in range(len(shapes))]
    assert set(ranks[:info.n_long]) == long_t
    fast = [elems[k].tensor for k in range(info.n_fast)]
    rest = [elems[k].tensor for k in range(info.n_fast, info.n_elem_items)]
    assert all(t in long_t for t in fast[:info.n_long_fast]) and not any(t in long_t for t in fast[info.n_long_fast:])
    assert all(t in long_t for t in rest[:info.n_long_rest]) and not any(t in long_t for t in rest[info.n_long_rest:])
    assert info.n_long_fast > 0 and info.n_long_rest > 0  # the 8M vector takes generic items
    # no split: every tensor long, the largest under 2^21 elements, a Lion plan
    for shp, opt in (([[1280, 11520], [1280, 11520]], 0), ([[1024, 2040], [8, 8]], 0), (shapes, 1)):
        _, info, _ = _plan_elems(shp, opt)
        assert (info.n_long, info.n_long_fast, info.n_long_rest) == (0, 0, 0), (shp, opt)
