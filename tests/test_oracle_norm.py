"""Pins the RMSNorm oracle (oracle/norm_oracle.py) independently of its own formula:

* against torch's ``rms_norm`` in float64 (a library routine: x · rsqrt(mean(x²) + eps) · w),
  in float64 end to end, for random rows, tiny and huge scales, and one-element rows;
* closed forms: a constant row c gives w · c / sqrt(c² + eps); eps = 0 makes the result
  invariant under scaling x; a 3-4 row gives (3, 4)/sqrt(12.5); an all-zero row gives 0 for
  eps > 0; Σ y² / H = ms / (ms + eps) for unit weights;
* the bias is added after the rounding of the normalised value (one more rounding);
* two norms in sequence read the first one's rounded output;
* the bf16 ulp distance helper on neighbours across zero and powers of two.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import norm_oracle as no


@pytest.mark.parametrize("H,scale", [(8, 1.0), (4096, 1.0), (5120, 1e-3), (777, 3e4), (1, 2.0)])
def test_matches_torch_rms_norm_float64(H, scale):
    g = torch.Generator().manual_seed(H)
    x = torch.randn(17, H, generator=g, dtype=torch.float64) * scale
    w = torch.randn(H, generator=g, dtype=torch.float64)
    for eps in (1e-6, 0.5):
        got = no.rms_norm_once(x, w, None, eps, torch.float64)
        want = F.rms_norm(x, (H,), w, eps)
        assert torch.allclose(got, want, rtol=1e-13, atol=0)


def test_closed_forms():
    H, eps = 64, 1e-6
    w = torch.linspace(-2, 2, H, dtype=torch.float64)
    for c in (0.5, -3.0, 1e-4):
        y = no.rms_norm_once(torch.full((1, H), c, dtype=torch.float64), w, None, eps, torch.float64)
        assert torch.allclose(y[0], w * c / math.sqrt(c * c + eps), rtol=1e-15, atol=0)
    x = torch.randn(5, H, dtype=torch.float64)
    a = no.rms_norm_once(x, w, None, 0.0, torch.float64)
    b = no.rms_norm_once(x * 1234.5, w, None, 0.0, torch.float64)
    assert torch.allclose(a, b, rtol=1e-14, atol=1e-15)
    y = no.rms_norm_once(torch.tensor([[3.0, 4.0]], dtype=torch.float64),
                         torch.ones(2, dtype=torch.float64), None, 0.0, torch.float64)
    assert torch.allclose(y, torch.tensor([[3.0, 4.0]], dtype=torch.float64) / math.sqrt(12.5))
    z = no.rms_norm_once(torch.zeros(2, H, dtype=torch.float64), w, None, eps, torch.float64)
    assert torch.equal(z, torch.zeros_like(z))
    y = no.rms_norm_once(x, torch.ones(H, dtype=torch.float64), None, 0.25, torch.float64)
    ms = (x * x).mean(-1)
    assert torch.allclose((y * y).mean(-1), ms / (ms + 0.25), rtol=1e-13)


def test_bias_after_rounding_and_chain():
    H = 8
    x = torch.tensor([[1.0, 2.0, 3.0, 4.0, 5.0, 6.0, 7.0, 8.0]], dtype=torch.bfloat16)
    w = torch.full((H,), 1.0, dtype=torch.bfloat16)
    b = torch.full((H,), 0.00390625, dtype=torch.bfloat16)       # 2^-8
    y0 = no.rms_norm_once(x, w, None, 0.0, torch.bfloat16)
    yb = no.rms_norm_once(x, w, b, 0.0, torch.bfloat16)
    want = (y0.to(torch.float64) + 0.00390625).to(torch.bfloat16)
    assert torch.equal(yb, want)
    # the first value: 1/sqrt(25.5) = 0.19803... -> bf16 0.1982421875; adding 2^-8 to the
    # rounded value gives 0.2021484375 (spacing 2^-10 in [0.125, 0.25))
    assert float(y0[0, 0]) == 0.1982421875 and float(yb[0, 0]) == 0.2021484375
    w2 = torch.linspace(0.5, 1.5, H).to(torch.bfloat16)
    chain = no.rms_norm(x, [(w, b, 1e-6), (w2, None, 1e-6)])
    two = no.rms_norm_once(no.rms_norm_once(x, w, b, 1e-6, torch.bfloat16), w2, None, 1e-6,
                           torch.bfloat16)
    assert torch.equal(chain, two)


def test_bf16_ulp_distance():
    a = torch.tensor([1.0, 1.0, -1.0, 0.0, 2.0, -0.0], dtype=torch.bfloat16)
    b = torch.tensor([1.0, 1.0078125, -1.0078125, 9.18355e-41, 1.9921875, 0.0], dtype=torch.bfloat16)
    assert no.bf16_ulp_distance(a, b).tolist() == [0, 1, 1, 1, 1, 0]
