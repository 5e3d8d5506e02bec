"""CPU oracle of the RMSNorm on the MoE input — TEST INFRASTRUCTURE ONLY.

Only tests/ may import this module (as the checker of the GPU path); the product package
``pisceslx_amd`` never imports it.

Restates, in float64, the RMSNorm the reference's CUDA path runs: ``YvRMSNorm.forward``
(model/core/norms.py:206-208) calls ``YvNorms._norm_forward`` (norms.py:992-1000), which on
CUDA uses ``fused_rms_norm`` (opss/kernels/fused_rms_norm.py:42-70, launched at :80-93):

* ``acc = Σ_h x_h²`` with x widened to fp32 (:56-60), ``rms = sqrt(acc / H + eps)`` (:62);
* ``y = (x / rms) * w`` computed in fp32 and stored once in x's dtype (:64-70; the output is
  ``empty_like(x)``, :83);
* a bias is added afterwards as a tensor op of x's dtype, one more rounding (norms.py:998-999).

Two norms in sequence (YvHybridBlock's ``norm_fusion`` then ``norm_mlp``,
model/core/hybrid.py:1359 and :1310) apply the second to the first one's rounded output.

The reference's torch fallback (norms.py:1001-1005, taken on CPU or without Triton) computes
``weight * x * rsqrt(mean(x²) + eps)`` in x's dtype with a rounding after every operation; it
is not what a CUDA host runs and is not restated here.

The oracle sums in float64, so its result can differ from an fp32 computation by one unit in
the last place of the output dtype where the exact value lies next to a rounding boundary;
tests compare within one bf16 ulp. Pinned in tests/test_oracle_norm.py against torch's own
``rms_norm`` in float64 and against closed forms.
"""
from __future__ import annotations

from typing import Optional, Sequence, Tuple

import torch

Norm = Tuple[torch.Tensor, Optional[torch.Tensor], float]


def rms_norm_once(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
                  eps: float, out_dtype: torch.dtype) -> torch.Tensor:
    """One norm (fused_rms_norm.py:56-70 and norms.py:998-999); x of any dtype, float64 math."""
    xd = x.to(torch.float64)
    H = xd.shape[-1]
    acc = (xd * xd).sum(-1, keepdim=True)
    rms = torch.sqrt(acc / H + float(eps))
    y = ((xd / rms) * weight.to(torch.float64)).to(out_dtype)
    if bias is not None:
        y = (y.to(torch.float64) + bias.to(torch.float64)).to(out_dtype)
    return y


def rms_norm(x: torch.Tensor, norms: Sequence[Norm]) -> torch.Tensor:
    """The norms in sequence, each rounded to x's dtype before the next one reads it."""
    y = x
    for w, b, eps in norms:
        y = rms_norm_once(y, w, b, eps, x.dtype)
    return y


def bf16_ulp_distance(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """|a - b| in units of the last place of bf16, as an integer distance between the ordered
    bit patterns (0 for identical values, 1 for neighbours)."""
    def key(t):
        u = t.contiguous().view(torch.int16).to(torch.int32) & 0xFFFF
        neg = (u & 0x8000) != 0
        return torch.where(neg, 0x8000 - (u & 0x7FFF), 0x8000 + u)
    return (key(a) - key(b)).abs()
