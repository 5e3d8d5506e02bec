"""Shared test helpers: oracle parameters of a workload, comparison metrics."""
import torch

from oracle.moe_oracle import params_from_workload as oracle_params  # noqa: F401


def cosine(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.double().reshape(-1)
    b = b.double().reshape(-1)
    return float((a @ b) / (a.norm() * b.norm() + 1e-300))


def max_abs(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.double() - b.double()).abs().max())
