"""GPU parity: the HIP step against the CPU oracle, bit for bit.

Every case steps the kaon_amd optimizer on cuda:0 and the oracle on the CPU
from the same seeded bytes and compares weights, momentum codes, scales and
the fp32 factored / 1-D state exactly (the HIP kernels implement the oracle's
canonical reduction order, so there is no tolerance).  Stochastic rounding is
compared exactly too: both sides draw the same Philox4x32-10 noise.

The oracle itself is pinned against the reference's outputs by
tests/test_oracle_golden.py and against closed forms by
tests/test_oracle_kat.py.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

import oracle as O  # noqa: E402
from golden_compare import CASES, CFG0  # noqa: E402
from gpu_cases import assert_same_as_oracle, oracle_case_run, run_gpu  # noqa: E402

GOLDEN = [k for k, c in CASES.items() if c["opt"] not in ("adamuon", "adapnm", "kprodigy")]  # own test files


@pytest.fixture(autouse=True, scope="module")
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")


@pytest.mark.parametrize("name", GOLDEN)
def test_golden_case_bit_exact(name):
    case = CASES[name]
    print(f"[gpu] golden case {name}", flush=True)
    oparams, _oopt, oeval = oracle_case_run(case)
    params, opt, evalp = run_gpu(case)
    assert_same_as_oracle(case, oparams, params, opt, evalp, oeval, label=name)


def test_configs0_bit_exact():
    """conv [320,320,3,3] + linear [1280,1280], beta1=0, SR, 10 steps."""
    print("[gpu] configs[0]", flush=True)
    oparams, _, _ = oracle_case_run(CFG0)
    params, opt, _ = run_gpu(CFG0)
    assert_same_as_oracle(CFG0, oparams, params, opt, label="cfg0")


def _case(opt, shapes, kwargs, steps=3, p="bf16", g="bf16", **kw):
    c = dict(steps=steps, seed=7, p_dtype=p, g_dtype=g, opt=opt, shapes=shapes, kwargs=kwargs)
    c.update(kw)
    return c


_MIX = [[640, 640, 3, 3], [1280, 2048], [5120, 640], [1280], [77, 33], [3, 5, 7], [1], [9, 1], [2, 2048 * 8],
        [13, 2880]]
# SDXL-shaped tensors of every row length of the benchmark set (640, 1280, 2048, 2880,
# 5120, 5760) plus 1-D, at sizes the oracle steps in about a second
_SDXL = [[640, 640, 3, 3], [1280, 1280], [256, 2048], [96, 5120], [320, 320, 3, 3], [64, 640, 3, 3], [5120, 640],
         [1280], [640], [77, 33]]
_PACKED = [[3, 1], [85, 7], [21, 9], [41, 20], [19, 33], [66, 100], [7, 129], [23, 256], [5, 257], [2, 3, 5], [40],
           [700, 9], [1000, 20]]
_VECS = [[5120], [1280], [20001], [1, 11520], [640], [320], [777], [2, 5120]]
EXTRA = {
    "ada_int8_mix": _case("adakaon", _MIX, dict(lr=1e-4, betas=(0.9, 0.999), momentum_dtype="int8")),
    "ada_4bit_mix_b64": _case("adakaon", _MIX, dict(lr=1e-4, betas=(0.9, 0.999), momentum_dtype="4bit",
                                                    momentum_4bit_block=64, weight_decay=0.01)),
    "ada_4bit_b3_rn": _case("adakaon", [[16, 9], [33], [5, 3, 2, 2]],
                            dict(lr=1e-3, betas=(0.8, 0.99), momentum_dtype="4bit", momentum_4bit_block=3,
                                 bf16_method="none")),
    "ada_bf16_kahan_mix": _case("adakaon", _MIX, dict(lr=1e-3, betas=(0.9, 0.999), momentum_dtype="bfloat16",
                                                      bf16_method="kahan", weight_decay=0.1)),
    "ada_f32_fp32_mix": _case("adakaon", _MIX, dict(lr=1e-3, betas=(0.9, 0.999), momentum_dtype="float32",
                                                    weight_decay=0.1, cautious=False), p="f32", g="f32"),
    "ada_nomom_nogc": _case("adakaon", _MIX, dict(lr=1e-4, betas=(0.0, 0.999), gradient_centralization=False,
                                                  eps=(0.0, 1e-3))),
    "ada_bf16p_f32g": _case("adakaon", [[64, 96], [40]], dict(lr=1e-3, momentum_dtype="int8"), g="f32"),
    "lion_int8_mix": _case("lion", _MIX, dict(lr=2e-4, betas=(0.95, 0.98), momentum_dtype="int8",
                                              weight_decay=0.1)),
    "lion_4bit_b256": _case("lion", _MIX, dict(lr=2e-4, betas=(0.95, 0.98), momentum_dtype="4bit",
                                               momentum_4bit_block=256, gradient_centralization=False)),
    "lion_f32": _case("lion", [[48, 40], [24]], dict(lr=1e-3, momentum_dtype="float32", bf16_method="none",
                                                     cautious=False), p="f32", g="f32"),
    "nekaon_4bit_b256": _case("nekaon", _MIX, dict(lr=1e-4, k=1.5, betas=(0.2, 0.999), momentum_dtype="4bit",
                                                   momentum_4bit_block=256), eval_train=True),
    # specialized bf16/SR kernels: fac == 1 and fac > 1, each codec, WD on and off
    "ada_bf16_sr_wd_clip_lo": _case("adakaon", _MIX, dict(lr=1e-3, momentum_dtype="bfloat16", weight_decay=0.05,
                                                          clip_threshold=0.1)),
    "ada_4bit_b128_clip_hi": _case("adakaon", _MIX, dict(lr=1e-4, momentum_dtype="4bit", clip_threshold=100.0)),
    "ada_int8_wd_clip_lo": _case("adakaon", _MIX, dict(lr=1e-4, momentum_dtype="int8", weight_decay=0.1,
                                                       clip_threshold=0.05)),
    "lion_bf16_gc_wd": _case("lion", _MIX, dict(lr=2e-4, momentum_dtype="bfloat16", weight_decay=0.1)),
    "lion_4bit_b64_gc": _case("lion", _MIX, dict(lr=2e-4, momentum_dtype="4bit", momentum_4bit_block=64)),
    "nekaon_int8_bf16": _case("nekaon", _MIX, dict(lr=1e-4, k=1.5, momentum_dtype="int8"), eval_train=True),
    "nekaon_4bit_b64_nowd": _case("nekaon", _MIX, dict(lr=1e-4, momentum_dtype="4bit", momentum_4bit_block=64,
                                                       weight_decay=0.0), eval_train=True),
    "nekaon_int8_f32": _case("nekaon", [[96, 40], [33], [4, 8, 3, 3]],
                             dict(lr=1e-3, k=1.5, momentum_dtype="int8"), p="f32", g="f32", eval_train=True),
    # BASELINE configs[3] as given: Nekaon k=1.5, beta1=0.2, wd 0.1, 4-bit blocks of 64 and
    # 256 (the 256-element blocks of the 640-, 2880- and 5760-element rows cross rows), grads
    # with 1 % Student-t(3) outliers that set the block absmax and drive the climb clamp;
    # eval/train at the end
    "cfg3_nekaon_4bit_b64": _case("nekaon", _SDXL, dict(lr=1e-4, k=1.5, betas=(0.2, 0.999), weight_decay=0.1,
                                                         momentum_dtype="4bit", momentum_4bit_block=64),
                                  outlier_frac=0.01, eval_train=True),
    "cfg3_nekaon_4bit_b256": _case("nekaon", _SDXL, dict(lr=1e-4, k=1.5, betas=(0.2, 0.999), weight_decay=0.1,
                                                          momentum_dtype="4bit", momentum_4bit_block=256),
                                   outlier_frac=0.01, eval_train=True),
    # Nekaon's keep count evaluates the cautious test for both neighbours the removal's
    # stochastic rounding can pick and draws the noise only where they disagree; a decay
    # of 50 on weights of 0.02 cancels the update often, so that branch runs too
    "nekaon_lazy_removal_ambiguous": _case("nekaon", [[320, 1280], [64, 640, 3, 3], [5120, 640]],
                                           dict(lr=1e-4, k=1.5, betas=(0.2, 0.999), weight_decay=50.0,
                                                momentum_dtype="4bit", momentum_4bit_block=64),
                                           steps=4, eval_train=True),
    # Nekaon with a param without a gradient on some steps (its climb is still removed and
    # re-added), all three on step 3
    "nekaon_gradless": _case("nekaon", [[320, 1280], [13, 2880], [640]],
                             dict(lr=1e-4, k=1.5, betas=(0.2, 0.999), momentum_dtype="4bit", momentum_4bit_block=64),
                             steps=4, no_grad={2: (1,), 3: (0, 1, 2)}, eval_train=True),
    # BASELINE configs[1] as given: Lion int8, betas=(0.95, 0.98), lr 2e-4, wd 0 (the
    # specialized kernel without weight decay), cautious, GC, SR
    "cfg1_lion_int8": _case("lion", _SDXL, dict(lr=2e-4, betas=(0.95, 0.98), momentum_dtype="int8"), steps=4),
    # rows of three chunks per lane whose third chunk fills 32, 16 or 2 lanes (C = 1280,
    # 1152, 1040), in wave groups of odd row counts (37 rows: waves of 6, 6, 1 and none;
    # 5 rows; 1 row), clipped
    "ada_int8_rows_1040_1280": _case("adakaon", [[37, 1280], [5, 1152], [1, 1280], [30, 1040], [1280]],
                                     dict(lr=1e-3, betas=(0.9, 0.999), momentum_dtype="int8", clip_threshold=0.05)),
    "lion_int8_rows_1040_1280": _case("lion", [[37, 1280], [5, 1152], [30, 1040]],
                                      dict(lr=2e-4, betas=(0.95, 0.98), momentum_dtype="int8")),
    # short rows side by side in a wave (rows of at most 32 chunks): 1 to 32 chunks per row
    # (lane groups of 1 to 32 lanes, some with lanes past the row), 1 to 64 rows per pass,
    # wave groups of 20 rows split over several passes, two slices ([85, 7]), ragged chunks;
    # [5, 257] (33 chunks) is the first length kept one row at a time; [700, 9] and [1000, 20]
    # span 3 and 4 runs of 320 rows (one column partial per run)
    "ada_int8_packed_rows_f32": _case("adakaon", _PACKED, dict(lr=1e-3, betas=(0.9, 0.999), momentum_dtype="int8",
                                                               weight_decay=0.05, clip_threshold=0.05),
                                      p="f32", g="f32"),
    "ada_bf16_rn_packed_rows": _case("adakaon", _PACKED, dict(lr=1e-3, momentum_dtype="bfloat16",
                                                              bf16_method="none")),
    "lion_int8_packed_rows_f32": _case("lion", _PACKED, dict(lr=2e-4, betas=(0.95, 0.98), momentum_dtype="int8"),
                                       p="f32", g="f32"),
    "nekaon_int8_packed_rows_f32": _case("nekaon", _PACKED, dict(lr=1e-4, k=1.5, momentum_dtype="int8"),
                                         p="f32", g="f32", steps=4),
    # items of one row (1-D tensors, a one-row matrix) shared by the four waves of the
    # phase-5/6 workgroup: int8 scales over the whole row, 4-bit blocks that cross
    # chunks (96) and blocks of whole chunks (64)
    "ada_int8_vectors": _case("adakaon", _VECS, dict(lr=1e-3, betas=(0.9, 0.999), momentum_dtype="int8",
                                                     weight_decay=0.05)),
    "ada_int8_vectors_f32": _case("adakaon", _VECS, dict(lr=1e-3, momentum_dtype="int8"), p="f32", g="f32"),
    "ada_4bit_b96_vectors": _case("adakaon", _VECS, dict(lr=1e-3, momentum_dtype="4bit", momentum_4bit_block=96)),
    "lion_4bit_b64_vectors": _case("lion", _VECS, dict(lr=2e-4, momentum_dtype="4bit", momentum_4bit_block=64)),
    "nekaon_int8_vectors": _case("nekaon", _VECS, dict(lr=1e-4, k=1.5, momentum_dtype="int8"), steps=4),
}


@pytest.mark.parametrize("name", sorted(EXTRA))
def test_extra_case_bit_exact(name):
    case = EXTRA[name]
    print(f"[gpu] extra case {name}", flush=True)
    oparams, _, oeval = oracle_case_run(case)
    params, opt, evalp = run_gpu(case)
    assert_same_as_oracle(case, oparams, params, opt, evalp, oeval, label=name)


def test_lora_bag_launch_bound_regime():
    """The reference's launch-bound proxy (benchmarks/proxy/harness.py:117-127): 512 fp32
    LoRA factors of [8, 16], Adakaon defaults (bf16 momentum, GC, cautious), three steps,
    bit for bit against the oracle."""
    case = _case("adakaon", [[8, 16]] * 512, dict(lr=1e-3, betas=(0.9, 0.999), momentum_dtype="bfloat16"),
                 p="f32", g="f32")
    print("[gpu] lora bag 512 x [8, 16]", flush=True)
    oparams, _, _ = oracle_case_run(case)
    params, opt, _ = run_gpu(case)
    assert_same_as_oracle(case, oparams, params, opt, label="lora_bag")


@pytest.mark.parametrize("variant", ["bf16_int8", "f32g_4bit"])
def test_rows_longer_than_16384(variant):
    """Factored rows of 17280, 23040 and 28672 elements (SDXL up-block convs [640,1920,3,3]
    and [1280,2560,3,3], a linear with 28672 inputs): the streamed-row kernels fold the
    column partial in LDS segments.  bf16 grads + int8 take the specialized phase-5/6
    kernel; fp32 grads + 4-bit (blocks crossing rows) the generic ones."""
    shapes = [[640, 1920, 3, 3], [1280, 2560, 3, 3], [96, 28672], [1920]]
    if variant == "bf16_int8":
        case = _case("adakaon", shapes, dict(lr=1e-4, betas=(0.9, 0.999), momentum_dtype="int8"), steps=2)
    else:
        case = _case("adakaon", shapes,
                     dict(lr=1e-4, betas=(0.9, 0.999), momentum_dtype="4bit", momentum_4bit_block=96,
                          weight_decay=0.01), steps=2, g="f32")
    print(f"[gpu] long rows {variant}", flush=True)
    oparams, _, _ = oracle_case_run(case)
    params, opt, _ = run_gpu(case)
    assert_same_as_oracle(case, oparams, params, opt, label=f"long_rows_{variant}")


def test_linear_of_28672_inputs():
    """A [4096, 28672] linear (117M elements, rows of 28672) through Adakaon int8, one step."""
    case = _case("adakaon", [[4096, 28672]], dict(lr=1e-4, betas=(0.9, 0.999), momentum_dtype="int8"), steps=1)
    print("[gpu] linear [4096, 28672]", flush=True)
    oparams, _, _ = oracle_case_run(case)
    params, opt, _ = run_gpu(case)
    assert_same_as_oracle(case, oparams, params, opt, label="linear_28672")


def test_sdxl_largest_conv_two_steps():
    """The largest SDXL tensor (conv [1280,1280,3,3], rows of 11520) through Adakaon int8."""
    case = _case("adakaon", [[1280, 1280, 3, 3]], dict(lr=1e-4, betas=(0.9, 0.999), momentum_dtype="int8"),
                 steps=2)
    print("[gpu] sdxl largest conv", flush=True)
    oparams, _, _ = oracle_case_run(case)
    params, opt, _ = run_gpu(case)
    assert_same_as_oracle(case, oparams, params, opt, label="conv1280")


# ----------------------------------------------------------------- primitives
def _lib():
    from kaon_amd import _lib

    return _lib.lib()


def _stream():
    return torch.cuda.current_stream().cuda_stream


def test_quant_int8_and_4bit_primitives_match_oracle():
    rng = np.random.default_rng(11)
    m = (rng.standard_normal((37, 301)) * np.exp(rng.standard_normal((37, 1)))).astype(np.float32)
    m[3] = 0.0
    m[5, 7] = np.float32(127.0 * 0.5)
    dm = torch.from_numpy(m).cuda()
    q = torch.empty(m.shape, dtype=torch.int8, device="cuda")
    sc = torch.empty(37, dtype=torch.float32, device="cuda")
    assert _lib().kaon_quant_int8(dm.data_ptr(), 37, 301, q.data_ptr(), sc.data_ptr(), _stream()) == 0
    oq, osc = O.quant_int8(m)
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy(), oq) and np.array_equal(sc.cpu().numpy(), osc)
    flat = m.reshape(-1)
    for block in (1, 7, 64, 128, 256, 4096):
        n = flat.size
        pk = torch.empty((n + 1) // 2, dtype=torch.uint8, device="cuda")
        s4 = torch.empty((n + block - 1) // block, dtype=torch.float32, device="cuda")
        src = torch.from_numpy(flat).cuda()
        assert _lib().kaon_quant_4bit(src.data_ptr(), n, block, pk.data_ptr(), s4.data_ptr(), _stream()) == 0
        opk, os4 = O.quant_4bit(flat, block)
        torch.cuda.synchronize()
        assert np.array_equal(pk.cpu().numpy(), opk), block
        assert np.array_equal(s4.cpu().numpy(), os4), block


def test_sr_noise_matches_oracle_philox():
    for (n, seed, step, tid, sid) in [(1000, 0, 1, 0, 1), (4099, 123456789, 77, 5, 2), (8, 2**32 - 1, 2**31, 1677, 0)]:
        out = torch.empty(n, dtype=torch.int16, device="cuda")
        assert _lib().kaon_sr_noise(out.data_ptr(), n, seed, step, tid, sid, _stream()) == 0
        want = O.sr_noise(n, seed, step, tid, sid)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint16), want)


def test_sr_round_bit_trick_matches_oracle_and_is_unbiased():
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(1 << 16).astype(np.float32),
                        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 3.3895e38, -3.3895e38, 1e-40], np.float32)])
    noise = rng.integers(0, 1 << 16, x.size).astype(np.uint16)
    dx, dn = torch.from_numpy(x).cuda(), torch.from_numpy(noise.view(np.int16)).cuda()
    out = torch.empty(x.size, dtype=torch.int16, device="cuda")
    assert _lib().kaon_sr_round(dx.data_ptr(), dn.data_ptr(), x.size, out.data_ptr(), _stream()) == 0
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint16), O.sr_round(x, noise))


def test_exact_division_helper_against_ieee_division():
    """div_r64 (fp64-reciprocal quotient) is used for every per-element division;
    check the quantizer's quotients against numpy's IEEE fp32 division on
    adversarial inputs (tie cases at code boundaries, wide exponent range)."""
    rng = np.random.default_rng(9)
    rows, cols = 64, 4096
    scale_src = np.exp(rng.uniform(-30, 30, (rows, 1))).astype(np.float32)
    m = (rng.uniform(-1, 1, (rows, cols)) * scale_src).astype(np.float32)
    # exact half-integer multiples of the scale -> rounding ties
    amax = np.abs(m).max(axis=1, keepdims=True)
    sc = (np.maximum(amax, np.float32(1e-12)) / np.float32(127.0)).astype(np.float32)
    m[:, :256] = (np.arange(-127.5, 0.5, 0.5, dtype=np.float32)[None, :256] * sc).astype(np.float32)
    dm = torch.from_numpy(m).cuda()
    q = torch.empty(m.shape, dtype=torch.int8, device="cuda")
    s = torch.empty(rows, dtype=torch.float32, device="cuda")
    assert _lib().kaon_quant_int8(dm.data_ptr(), rows, cols, q.data_ptr(), s.data_ptr(), _stream()) == 0
    torch.cuda.synchronize()
    s_np = s.cpu().numpy()
    ref = np.clip(np.rint(m / s_np[:, None]), -127, 127).astype(np.int8)
    assert np.array_equal(q.cpu().numpy(), ref)


def test_injected_noise_path():
    """Injected per-element noise replaces Philox on both sides (the harness the
    reference goldens were made with)."""
    from cases import param_values

    case = _case("adakaon", [[24, 40], [17]], dict(lr=1e-3, momentum_dtype="int8"), steps=1)
    rng = np.random.default_rng(3)
    noise = {i: [None, rng.integers(0, 1 << 16, int(np.prod(s))).astype(np.uint16), None]
             for i, s in enumerate(case["shapes"])}
    from golden_compare import dt, group_for
    from cases import grad_values

    g = group_for(case)
    oparams = [O.make_param(s, tensor_id=i, p_values=param_values(case, i)) for i, s in enumerate(case["shapes"])]
    oopt = O.OracleOptimizer(oparams, "adakaon", g, seed=case["seed"])
    for i, prm in enumerate(oparams):
        prm.g = O.f32_to_bf16(grad_values(case, i, 1)).reshape(prm.shape)
    oopt.step(noise=noise)
    from gpu_cases import make_opt

    params = [torch.nn.Parameter(torch.from_numpy(param_values(case, i)).cuda().bfloat16())
              for i in range(len(case["shapes"]))]
    opt = make_opt(case, params)
    for i, p in enumerate(params):
        opt._inject_noise[p] = [None, torch.from_numpy(noise[i][1].view(np.int16)).cuda(), None]
        p.grad = torch.from_numpy(grad_values(case, i, 1)).cuda().bfloat16()
    opt.step()
    torch.cuda.synchronize()
    assert_same_as_oracle(case, oparams, params, opt, label="inject")
    _ = dt
