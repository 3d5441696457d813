"""Bias of the library's bf16 stochastic rounding over 1e7 samples.

The SR write of every step adds a 16-bit Philox4x32-10 noise word to the fp32
bit pattern and clears the low half (the `_add_stochastic_bf16_` bit trick,
src/kaon/_stochastic_rounding.py:88-103).  For a value v whose low 16 bits are
f, it rounds up with probability f / 65536 exactly when the noise is uniform,
so E[SR(v)] = v.  This test runs the library's own noise stream
(kaon_sr_noise, the generator the fused step uses) through its rounding
(kaon_sr_round) for 10 values x 1e6 samples each.  It reports the bias of the
sample mean in units of the bf16 ulp, and asserts it is within 6 standard
errors of zero for every value (a biased rounding, e.g. round-to-nearest or a
noise word missing its top bit, is off by more than 0.1 ulp).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

N_PER = 1_000_000
FRACS = [1, 4097, 16384, 21845, 32767, 32768, 43690, 49152, 61439, 65535]  # low 16 bits of v


@pytest.fixture(autouse=True, scope="module")
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")


def _lib():
    from kaon_amd import _lib

    return _lib.lib()


def test_sr_bias_over_1e7_samples():
    rng = np.random.default_rng(2024)
    # bf16 grid points over several binades, both signs; v = grid point + f / 65536 ulp
    hi = (rng.integers(0x3C00, 0x4300, len(FRACS)) | (rng.integers(0, 2, len(FRACS)) << 15)).astype(np.uint32)
    vbits = (hi << 16) | np.array(FRACS, dtype=np.uint32)
    v = vbits.view(np.float32)
    ulp = np.abs((((hi + 1) << 16).view(np.float32)) - ((hi << 16).view(np.float32))).astype(np.float64)
    n = N_PER * len(FRACS)
    print(f"[gpu] sr bias: {len(FRACS)} values x {N_PER} samples", flush=True)
    x = torch.from_numpy(np.repeat(v, N_PER)).cuda()
    noise = torch.empty(n, dtype=torch.int16, device="cuda")
    out = torch.empty(n, dtype=torch.int16, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    assert _lib().kaon_sr_noise(noise.data_ptr(), n, 0x5EED, 7, 3, 1, s) == 0
    assert _lib().kaon_sr_round(x.data_ptr(), noise.data_ptr(), n, out.data_ptr(), s) == 0
    torch.cuda.synchronize()
    bits = out.to(torch.int32).bitwise_and(0xFFFF).bitwise_left_shift(16)
    vals = bits.view(torch.float32).double().view(len(FRACS), N_PER)
    mean = vals.mean(dim=1).cpu().numpy()
    bias_ulp = (mean - v.astype(np.float64)) / ulp
    p = np.array(FRACS, dtype=np.float64) / 65536.0
    se_ulp = np.sqrt(p * (1 - p) / N_PER)
    # the rounded values are exactly the two neighbours
    up = ((bits.view(torch.float32).double().view(len(FRACS), N_PER) - torch.from_numpy(v.astype(np.float64))
           .cuda()[:, None]).abs().cpu().numpy().max(axis=1))
    assert (up <= ulp * (1 + 1e-12)).all()
    for f, b, e in zip(FRACS, bias_ulp, se_ulp):
        print(f"  low16={f:5d}  P(up)={f / 65536:.6f}  bias={b:+.3e} ulp  (s.e. {e:.1e})", flush=True)
    print(f"  overall mean |bias| = {np.abs(bias_ulp).mean():.3e} ulp over {n} samples", flush=True)
    assert (np.abs(bias_ulp) <= 6 * se_ulp + 1e-12).all(), bias_ulp
