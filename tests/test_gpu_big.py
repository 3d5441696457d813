"""Tensors of 2^31 elements and more (up to 2^32 - 1) on the GPU.

The oracle cannot step 2^31 elements in a test's time, so these tests check
the large-offset path against the planned path of smaller tensors, bit for bit,
where the step is row-local: Lion with cautious masking off takes each row's
GC mean, its int8 scale (or its 4-bit blocks, when they do not cross the split)
and its injected SR noise from that row alone, so the big tensor and the same
rows as two tensors of fewer than 2^31 elements (which the parity suite pins
against the oracle) must give identical weights and momentum.  Adakaon's
factored statistics couple the rows; its row and column state after a step is
compared with a float64 torch computation of the same EMA.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
R, C = 131073, 16384  # 2^31 + 2^14 elements


@pytest.fixture(autouse=True, scope="module")
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")


def _data(seed):
    gen = torch.Generator(device=DEV)
    gen.manual_seed(seed)
    p = (torch.randn(R, C, device=DEV, generator=gen) * 0.02).bfloat16()
    grads = [(torch.randn(R, C, device=DEV, generator=gen) * 1e-3).bfloat16() for _ in range(2)]
    noise = torch.randint(-(1 << 15), 1 << 15, (R * C,), device=DEV, dtype=torch.int16, generator=gen)
    return p, grads, noise


@pytest.mark.parametrize("momentum_dtype,block,split", [("int8", 128, 65536), ("4bit", 128, 65536),
                                                         ("4bit", 96, 65535)])
def test_lion_big_tensor_equals_its_rows_as_two_tensors(momentum_dtype, block, split):
    from kaon_amd import Lion

    print(f"[gpu] big Lion {momentum_dtype} block {block}", flush=True)
    assert (split * C) % block == 0  # 4-bit blocks of the pieces start where the big tensor's do
    p0, grads, noise = _data(11)
    kw = dict(lr=2e-4, betas=(0.95, 0.98), weight_decay=0.1, momentum_dtype=momentum_dtype,
              momentum_4bit_block=block, cautious=False, gradient_centralization=True,
              bf16_method="stochastic_rounding")
    head = p0[:4].clone()
    big = torch.nn.Parameter(p0.clone())
    opt_big = Lion([big], **kw)
    opt_big._inject_noise[big] = [None, noise, None]
    parts = [torch.nn.Parameter(p0[:split].clone()), torch.nn.Parameter(p0[split:].clone())]
    del p0
    opt_parts = Lion(parts, **kw)
    opt_parts._inject_noise[parts[0]] = [None, noise[: split * C], None]
    opt_parts._inject_noise[parts[1]] = [None, noise[split * C:], None]
    for g in grads:
        # copies: each step leaves its p.grad centralized in place
        parts[0].grad, parts[1].grad = g[:split].clone(), g[split:].clone()
        big.grad = g
        opt_big.step()
        opt_parts.step()
    torch.cuda.synchronize()
    assert torch.equal(big[:split], parts[0]) and torch.equal(big[split:], parts[1])
    sb = opt_big.state[big]
    s0, s1 = opt_parts.state[parts[0]], opt_parts.state[parts[1]]
    mb = sb["m"].reshape(-1)
    n0 = s0["m"].numel()
    assert torch.equal(mb[:n0], s0["m"].reshape(-1)) and torch.equal(mb[n0:], s1["m"].reshape(-1))
    sc = sb["m_scale"].reshape(-1)
    k0 = s0["m_scale"].numel()
    assert torch.equal(sc[:k0], s0["m_scale"].reshape(-1)) and torch.equal(sc[k0:], s1["m_scale"].reshape(-1))
    # the steps moved the weights: the comparison is not of untouched copies
    assert not torch.equal(big[:4], head)


def test_adakaon_big_tensor_factored_state():
    """Rows past 2^31 / C elements: the row / column EMA of the step (GC'd grads,
    means rounded to bf16 first) against float64 torch, within the fp32 summation
    error of 131073-row column sums; the weights finite, and most of them moved."""
    from kaon_amd import Adakaon

    print("[gpu] big Adakaon int8", flush=True)
    p0, grads, _noise = _data(12)
    del _noise
    g = grads[0]
    del grads
    p = torch.nn.Parameter(p0.clone())
    # fused=True leaves p.grad as given, so the restatement below reads the raw grads
    opt = Adakaon([p], lr=1e-3, betas=(0.9, 0.999), weight_decay=0.0, momentum_dtype="int8", fused=True)
    p.grad = g
    opt.step()
    torch.cuda.synchronize()
    st = opt.state[p]
    # float64 restatement of the factored EMA from zero state (adakaon.py:975-995, _factored.py:26-83)
    row = torch.empty(R, dtype=torch.float64, device=DEV)
    col = torch.zeros(C, dtype=torch.float64, device=DEV)
    b2 = 0.999
    for r0 in range(0, R, 8192):
        gb = g[r0:r0 + 8192].double()
        mu = gb.mean(dim=1, keepdim=True).float().bfloat16().double()
        gc = (gb - mu).float().bfloat16().double()
        q = gc * gc + 1e-30
        row[r0:r0 + 8192] = q.mean(dim=1) * (1 - b2)
        col += q.sum(dim=0)
    col = col / R * (1 - b2)
    got_row = st["row"].double()
    got_col = st["col"].double()
    assert torch.allclose(got_row, row, rtol=1e-4, atol=0), float(((got_row - row) / row).abs().max())
    assert torch.allclose(got_col, col, rtol=1e-4, atol=0), float(((got_col - col) / col).abs().max())
    assert torch.isfinite(p.detach()).all()
    moved = float((p.detach() != p0).float().mean())
    assert moved > 0.5, moved
