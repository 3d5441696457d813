"""Synthetic SDXL-UNet-shaped parameter sets for the benchmark and scale tests.

The shape vocabulary is BASELINE's configs[1]: conv [C_out, C_in, 3, 3] with
C in {320, 640, 1280}, linears [1280|2048|5120 x 640|1280|2048|5120] and 1-D
norm/bias vectors; the counts follow SDXL's block structure: 1,678 tensors,
2,664,150,400 params (74.5 % of them in tensors above 2M elements, the ones the
reference's foreach path steps one by one, src/kaon/adakaon.py:765-791).

Inputs are generated on the device, one torch generator per tensor keyed by
(seed, tensor index): weights N(0, 0.02^2) (the reference's ktune convention,
src/kaon/tune.py:72) and grads N(0, sigma^2) with log10(sigma) ~ U(-5, -2) per
tensor, both rounded to bf16.
"""
from __future__ import annotations

import numpy as np
import torch

SDXL_SHAPES: list[tuple[tuple[int, ...], int]] = [
    # linear
    ((1280, 1280), 368), ((1280, 2048), 130), ((5120, 1280), 120), ((1280, 5120), 60),
    ((5120, 640), 20), ((2048, 640), 20), ((1280, 640), 40),
    # conv
    ((1280, 1280, 3, 3), 22), ((640, 640, 3, 3), 10), ((320, 320, 3, 3), 8), ((1280, 640, 3, 3), 2),
    ((640, 1280, 3, 3), 3), ((640, 320, 3, 3), 2), ((320, 640, 3, 3), 3),
    # 1-D
    ((1280,), 580), ((5120,), 140), ((640,), 120), ((320,), 30),
]


def sdxl_shapes() -> list[tuple[int, ...]]:
    """The 1,678 shapes, largest first within each kind, kinds interleaved as listed."""
    out: list[tuple[int, ...]] = []
    for shape, count in SDXL_SHAPES:
        out.extend([shape] * count)
    return out


def n_params(shapes: list[tuple[int, ...]]) -> int:
    return int(sum(int(np.prod(s)) for s in shapes))


def grad_sigmas(n: int, seed: int = 0) -> np.ndarray:
    rng = np.random.default_rng([seed, 0x5D])
    return (10.0 ** rng.uniform(-5.0, -2.0, n)).astype(np.float64)


@torch.no_grad()
def make_params(shapes: list[tuple[int, ...]], device: torch.device, seed: int = 0,
                dtype: torch.dtype = torch.bfloat16, outlier_frac: float = 0.0) -> list[torch.nn.Parameter]:
    """Params with .grad set.  ``outlier_frac`` replaces that fraction of each
    grad's elements by Student-t(3) draws scaled by the tensor's sigma."""
    sig = grad_sigmas(len(shapes), seed)
    params = []
    for i, s in enumerate(shapes):
        gen = torch.Generator(device=device)
        gen.manual_seed(seed * 1_000_003 + i)
        p = (torch.randn(s, generator=gen, device=device, dtype=torch.float32) * 0.02).to(dtype)
        g = torch.randn(s, generator=gen, device=device, dtype=torch.float32) * float(sig[i])
        if outlier_frac > 0:
            mask = torch.rand(s, generator=gen, device=device) < outlier_frac
            # Student-t(3) = N / sqrt(chi2_3 / 3)
            z = torch.randn(s, generator=gen, device=device)
            chi = sum(torch.randn(s, generator=gen, device=device) ** 2 for _ in range(3)) / 3.0
            g = torch.where(mask, z / chi.sqrt() * float(sig[i]), g)
        prm = torch.nn.Parameter(p)
        prm.grad = g.to(dtype)
        params.append(prm)
    return params
