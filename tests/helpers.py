"""Shared test helpers: oracle parameters of a workload, comparison metrics."""
import numpy as np
import torch

from oracle import moe_oracle
from pisceslx_amd.workloads import Workload


def oracle_params(w: Workload) -> moe_oracle.LayerParams:
    cpu = w.experts.to("cpu")
    spec = w.spec
    pred = None if w.pred is None else tuple(t.detach().cpu() for t in w.pred)
    return moe_oracle.LayerParams(
        hidden=spec.hidden, ffn=spec.ffn, num_experts=spec.num_experts, num_shared=spec.num_shared,
        top_k=spec.top_k, gate_weight=w.gate_weight.cpu(), pred=pred,
        bias=None if w.expert_bias is None else w.expert_bias.cpu(),
        fixed_shape_mode=spec.fixed_shape_mode, dynamic_capacity=not spec.fixed_shape_mode,
        capacity_factor=1.0, min_capacity=4,
        mix_param=None if w.shared_expert_weight is None else w.shared_expert_weight.cpu(),
        expert_fn=lambda i: cpu.dequantize(i, torch.float32))


def cosine(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.double().reshape(-1)
    b = b.double().reshape(-1)
    return float((a @ b) / (a.norm() * b.norm() + 1e-300))


def max_abs(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.double() - b.double()).abs().max())
