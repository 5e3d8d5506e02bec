"""RMSNorm of the MoE input and the MoE half of the hybrid block, over libyvmoe.

YvRMSNorm mirrors model/core/norms.py:178-208 (constructor, parameter names, forward) and
computes what the reference's CUDA path computes, the fused kernel of
opss/kernels/fused_rms_norm.py:42 reached through YvNorms._norm_forward
(model/core/norms.py:992-1000): per row rms = sqrt(Σx²/H + eps) with an fp32 sum,
(x / rms) * weight rounded once to x's dtype, then + bias rounded again.

YvHybridBlockMLP holds the submodules of YvHybridBlock (model/core/hybrid.py:1206-1221) that
surround its MoE layer, under the block's own names (norm_fusion, norm_mlp, mlp,
residual_scale_mlp), and runs the block's MLP half (hybrid.py:1358-1366 with _forward_mlp
:1309-1317): the two norms in one native pass, the MoE layer, then the scaled residual.
"""
from __future__ import annotations

from typing import Any, Optional

import torch
import torch.nn as nn

from .functional import rms_norm
from .layer import YvDeepSeekMoELayer


class YvRMSNorm(nn.Module):
    """YvRMSNorm (model/core/norms.py:178-208) on the native kernel; weight and bias in x's dtype."""

    def __init__(self, dim: int, eps: float = 1e-6, use_bias: bool = False,
                 device: Optional[torch.device] = None, dtype: Optional[torch.dtype] = None):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim, device=device, dtype=dtype))
        self.use_bias = use_bias
        if use_bias:
            self.bias = nn.Parameter(torch.zeros(dim, device=device, dtype=dtype))
        else:
            self.register_parameter("bias", None)

    def reset_parameters(self):
        nn.init.ones_(self.weight)
        if self.use_bias and self.bias is not None:
            nn.init.zeros_(self.bias)

    def norm_params(self):
        return (self.weight.detach(), None if self.bias is None else self.bias.detach(), self.eps)

    @torch.no_grad()
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return rms_norm(x.contiguous(), [self.norm_params()])


def rms_norm_chain(x: torch.Tensor, first: YvRMSNorm, second: YvRMSNorm) -> torch.Tensor:
    """second(first(x)) in one pass over x (each norm rounded to x's dtype, as two calls round)."""
    return rms_norm(x.contiguous(), [first.norm_params(), second.norm_params()])


class YvHybridBlockMLP(nn.Module):
    """The MoE half of YvHybridBlock (model/core/hybrid.py:1206-1221, :1309-1317, :1358-1366).

    forward(hybrid_out, modal_id) -> (output, aux_loss) with
    output = hybrid_out + residual_scale_mlp * mlp(norm_mlp(norm_fusion(hybrid_out))), as the
    block computes in eval mode (residual dropout inactive). The two norms run as one kernel.
    """

    def __init__(self, cfg: Any, device=None, dtype=None, weight_format: Optional[str] = None,
                 router: Optional[str] = None):
        super().__init__()
        H = cfg.hidden_size
        self.norm_fusion = YvRMSNorm(H, device=device, dtype=dtype)
        self.mlp = YvDeepSeekMoELayer(cfg, device=device, dtype=dtype, weight_format=weight_format,
                                      router=router)
        self.norm_mlp = YvRMSNorm(H, device=device, dtype=dtype)
        self.residual_scale_mlp = nn.Parameter(
            torch.ones(1, device=device, dtype=dtype) * (2.0 * cfg.n_layer) ** -0.5)

    @torch.no_grad()
    def forward(self, hybrid_out: torch.Tensor, modal_id: Optional[torch.Tensor] = None):
        x_norm = rms_norm_chain(hybrid_out, self.norm_fusion, self.norm_mlp)
        result = self.mlp(x_norm, modal_id=modal_id)
        mlp_out, aux_loss = result if isinstance(result, (tuple, list)) else (result, None)
        if aux_loss is None:
            aux_loss = torch.tensor(0.0, device=hybrid_out.device, dtype=hybrid_out.dtype)
        return hybrid_out + self.residual_scale_mlp * mlp_out, aux_loss
