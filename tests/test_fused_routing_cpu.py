"""Which params' p.grad Adakaon(fused=True) leaves centralized (CPU, host logic only).

The reference's fused Adakaon partitions a group (``_fused_partition``,
src/kaon/adakaon.py:437-468) into one-block, big (chunked), 1-D and native
params; only the native ones go through ``centralize_grads_`` (in place on
p.grad, adakaon.py:396-401), and that touches params of 2 dims or more.
``fused_routes_native`` restates the partition's native branch; these cases
follow its conditions one by one.
"""
import pytest
import torch

from kaon_amd.adakaon import fused_routes_native


def _p(shape, dtype=torch.bfloat16):
    p = torch.nn.Parameter(torch.zeros(shape, dtype=dtype))
    p.grad = torch.zeros(shape, dtype=dtype)
    return p


def _group(**kw):
    g = dict(momentum_dtype="int8", betas=(0.9, 0.999), bf16_method="stochastic_rounding")
    g.update(kw)
    return g


CASES = [
    # (shape, dtype, group kwargs, native?)
    ([24, 40], torch.bfloat16, {}, False),                                  # one-block matrix
    ([16, 8, 3, 3], torch.bfloat16, {}, True),                              # conv, int8 momentum
    ([16, 8, 3, 3], torch.bfloat16, dict(momentum_dtype="4bit"), True),     # conv, 4-bit momentum
    ([16, 8, 3, 3], torch.bfloat16, dict(momentum_dtype="bfloat16"), False),
    ([16, 8, 3, 3], torch.float32, dict(momentum_dtype="float32"), False),
    ([7, 9], torch.bfloat16, dict(momentum_dtype="4bit"), True),            # one-block 4-bit, odd width
    ([7, 10], torch.bfloat16, dict(momentum_dtype="4bit"), False),
    ([600, 301], torch.bfloat16, dict(momentum_dtype="4bit"), False),       # big: the odd-width rule is one-block only
    ([600, 300], torch.bfloat16, {}, False),                                # 1024 x 512 > 2^17: big
    ([256, 512], torch.bfloat16, {}, False),                                # 2^17 exactly: one-block
    ([24, 40], torch.bfloat16, dict(betas=(0.0, 0.999)), True),             # no momentum
    ([24, 40], torch.bfloat16, dict(bf16_method="kahan"), True),            # bf16 without SR
    ([24, 40], torch.bfloat16, dict(bf16_method="none"), True),
    ([24, 40], torch.float32, dict(bf16_method="kahan"), False),            # fp32 params: SR irrelevant
    ([24, 40], torch.float16, {}, True),                                    # fp16: native
    ([33], torch.bfloat16, {}, False),                                      # 1-D: never centralized
    ([33], torch.bfloat16, dict(betas=(0.0, 0.999)), False),
]


@pytest.mark.parametrize("shape,dtype,kw,native", CASES)
def test_fused_partition_native_branch(shape, dtype, kw, native):
    assert fused_routes_native(_p(shape, dtype), _group(**kw)) is native


def test_tile_cap_moves_the_one_block_limit():
    p = _p([600, 300])
    assert fused_routes_native(p, _group(), tile_cap=1 << 20) is False       # now one-block
    q = _p([7, 9])
    assert fused_routes_native(q, _group(momentum_dtype="4bit"), tile_cap=8) is False  # now big: no odd rule
