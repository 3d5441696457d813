"""Known-answer and closed-form checks that pin the oracle's primitives.

Philox4x32-10: the Random123 published known-answer vectors.  Codecs: the
closed forms of src/kaon/_momentum_codec.py:72-200 (tie cases, floors,
nibble range, zero state) and the reference's own invariants
(tests/test_momentum_codec.py:100-153 in the reference).  SR: the bit trick
of src/kaon/_stochastic_rounding.py:70-103 on hand-built cases.
"""
import numpy as np
import pytest

import oracle as O


@pytest.mark.parametrize("ctr,key,expect", [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
])
def test_philox_random123_kat(ctr, key, expect):
    assert tuple(int(x) for x in O.philox4x32_10(ctr, key)) == expect


def test_sr_noise_layout():
    """Element e of a chunk takes 16-bit half (e%8) of Philox(ctr=(e/8,0,tid,stream), key=(seed,step))."""
    n = 20
    noise = O.sr_noise(n, seed=7, step=3, tensor_id=5, stream=1)
    for e in range(n):
        out = O.philox4x32_10((e // 8, 0, 5, 1), (7, 3))
        w = e % 8
        assert noise[e] == (int(out[w // 2]) >> (16 * (w % 2))) & 0xFFFF


def test_noise_is_uniform_16bit():
    noise = O.sr_noise(1 << 20, seed=0, step=1, tensor_id=0, stream=1).astype(np.float64)
    assert abs(noise.mean() - 32767.5) < 100
    hist = np.bincount((noise // 4096).astype(np.int64), minlength=16)
    assert hist.min() > 0.9 * hist.mean()


def test_sr_bit_trick_cases():
    one = np.float32(1.0)
    ulp = np.float32(2.0 ** -7)  # bf16 ulp at 1.0
    x = np.array([one + ulp / 4], dtype=np.float32)
    lo, hi = O.f32_to_bf16(np.array([one]))[0], O.f32_to_bf16(np.array([one + ulp]))[0]
    # noise below 0xC000 keeps the truncation, at/above rounds up (1/4 of the gap)
    assert O.sr_round(x, np.array([0xBFFF], np.uint16))[0] == lo
    assert O.sr_round(x, np.array([0xC000], np.uint16))[0] == hi
    # negative values: magnitude rounds up with the same probability
    xn = -x
    assert O.sr_round(xn, np.array([0xC000], np.uint16))[0] == (hi | 0x8000)
    # exact bf16 values never move
    exact = O.bf16_to_f32(np.array([0x3F80, 0xBF80, 0x0000, 0x4049], np.uint16))
    for nz in (0, 0x7FFF, 0xFFFF):
        assert np.array_equal(O.sr_round(exact, np.full(4, nz, np.uint16)),
                              np.array([0x3F80, 0xBF80, 0x0000, 0x4049], np.uint16))
    # the largest finite value can carry into inf
    big = np.array([np.float32(3.3895e38)], dtype=np.float32)
    r = O.sr_round(big, np.array([0xFFFF], np.uint16))[0]
    assert r in (0x7F7F, 0x7F80)


def test_sr_unbiased_statistic():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(4096).astype(np.float32)
    acc = np.zeros_like(x, dtype=np.float64)
    for s in range(300):
        acc += O.bf16_to_f32(O.sr_round(x, O.sr_noise(x.size, 11, s, 0, 1)))
    assert np.abs(acc / 300 - x).mean() < 5e-4  # the reference's own bound


def test_int8_closed_form_and_ties():
    scale_src = np.float32(127.0)  # absmax 127 -> scale exactly 1.0
    m = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -126.5, 3.49]], dtype=np.float32)
    q, sc = O.quant_int8(m)
    assert sc[0] == np.float32(1.0)
    assert q.tolist() == [[127, 0, 2, 2, 0, -2, -126, 3]]  # round half to even
    z, zs = O.quant_int8(np.zeros((3, 5), np.float32))
    assert (z == 0).all() and np.all(zs == np.float32(1e-12) / scale_src)
    # 1-D: one scalar scale over the whole tensor
    q1, s1 = O.quant_int8(np.array([1.0, -4.0, 2.0], np.float32))
    assert s1.shape == (1,) and s1[0] == np.float32(4.0) / scale_src
    # round trip error <= step/2 per row
    rng = np.random.default_rng(0)
    m = (rng.standard_normal((16, 50)) * np.exp(rng.standard_normal((16, 1)))).astype(np.float32)
    q, sc = O.quant_int8(m)
    deq = O.dequant("int8", q, sc, m.shape)
    assert np.all(np.abs(deq - m) <= sc[:, None] / 2 * (1 + 1e-6))
    assert np.abs(q).max() <= 127


def test_4bit_closed_form():
    m = np.array([7.0, 0.5, 1.5, -2.5, 3.5, -7.0, 0.0, 6.5, 1.0], dtype=np.float32)
    pk, sc = O.quant_4bit(m, 4)
    assert np.allclose(sc, [7.0 / 7.0, 7.0 / 7.0, 1.0 / 7.0])
    nib = [(pk[i >> 1] >> (4 * (i & 1))) & 0xF for i in range(m.size)]
    assert nib == [15, 8, 10, 6, 12, 1, 8, 14, 15]
    assert pk[-1] >> 4 == 0  # odd numel: dangling high nibble is zero
    rng = np.random.default_rng(3)
    m = (rng.standard_normal(257) * 50).astype(np.float32)
    pk, sc = O.quant_4bit(m, 128)
    nibs = np.stack([pk & 0xF, pk >> 4], 1).reshape(-1)[:257]
    assert nibs.min() >= 1 and nibs.max() <= 15
    deq = O.dequant("4bit", pk, sc, (257,), 128)
    step = np.repeat(sc, 128)[:257]
    assert np.all(np.abs(deq - m) <= step / 2 * (1 + 1e-6))


def test_fresh_4bit_state_is_zero():
    st = O.make_param((5, 7), p_values=np.zeros((5, 7)))
    O.init_state(st, "adakaon", dict(betas=(0.9, 0.999), momentum_dtype="4bit", momentum_4bit_block=128))
    assert (st.state["m"] == 0x88).all() and (st.state["m_scale"] == 1.0).all()
    assert np.all(O.dequant("4bit", st.state["m"], st.state["m_scale"], (5, 7), st.state["m_block"]) == 0)


def test_csum_matches_exact_sum_closely():
    rng = np.random.default_rng(5)
    for n in (1, 7, 8, 9, 100, 2049, 11520, 1 << 18):
        x = rng.standard_normal(n).astype(np.float32)
        assert abs(float(O.csum(x)) - x.astype(np.float64).sum()) <= 1e-6 * np.abs(x).sum() + 1e-30
    # integers are summed exactly
    x = np.ones(100003, np.float32)
    assert O.csum(x) == np.float32(100003)


def test_csum_order_definition():
    """Brute force of the canonical order on a case where order matters."""
    x = np.zeros(2048 + 8, np.float32)
    x[0] = 1e8
    x[1:8] = 1.0       # lane 0 sequential: 1e8 + 1 + ... absorbed one at a time
    x[2048] = -1e8     # chunk 256 -> lane 0 again, after the first chunk
    x[8] = 1.0         # lane 1
    got = float(O.csum(x))
    # lane 0: ((1e8 + 1)+...+1) = 1e8 (each +1 rounds away), then -1e8 -> 0; lane 1: 1
    assert got == 1.0
