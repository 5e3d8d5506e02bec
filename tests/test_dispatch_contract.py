"""Host-side contract of the dispatch operator mirror (pisceslx_amd/dispatch.py), on the CPU:
the checks that run before any device work.

* training semantics: the reference operator runs its experts' dropout and builds an autograd
  graph in training mode (opss/infer/fused_moe.py:103-111 -> model/moe/expert.py:484-489);
  the MI355X operator is an inference forward, so the module in training mode, an expert in
  training mode, or inputs that require grad under autograd raise NotImplementedError instead
  of returning a detached output;
* the size check of fused_moe.py:76-82 raises ValueError.
"""
import pytest
import torch
import torch.nn as nn

from pisceslx_amd.dispatch import PiscesLxFusedMoEDispatch, PiscesLxFusedMoe


class _SwiGLU(nn.Module):
    def __init__(self, H=8, F=16):
        super().__init__()
        self.gate_proj = nn.Linear(H, F, bias=False)
        self.up_proj = nn.Linear(H, F, bias=False)
        self.down_proj = nn.Linear(F, H, bias=False)
        self.dropout = nn.Dropout(0.1)


def _inputs(N=4, k=2, E=3, H=8):
    x = torch.randn(N, H)
    w = torch.full((N, k), 1.0 / k)
    idx = torch.randint(0, E, (N, k))
    return x, w, idx


def test_module_in_training_mode_raises():
    x, w, idx = _inputs()
    experts = nn.ModuleList([_SwiGLU() for _ in range(3)]).eval()
    m = PiscesLxFusedMoEDispatch(3, 2)
    assert m.training
    with pytest.raises(NotImplementedError, match="inference"):
        m(x, w, idx, experts)


def test_expert_in_training_mode_raises():
    x, w, idx = _inputs()
    experts = nn.ModuleList([_SwiGLU() for _ in range(3)]).eval()
    experts[1].train()
    m = PiscesLxFusedMoEDispatch(3, 2).eval()
    with pytest.raises(NotImplementedError, match="training mode"):
        m(x, w, idx, experts)
    with pytest.raises(NotImplementedError, match="training mode"):
        PiscesLxFusedMoe.fused_moe_dispatch(x, w, idx, experts, 3, 2)


def test_inputs_requiring_grad_raise_under_autograd():
    x, w, idx = _inputs()
    experts = nn.ModuleList([_SwiGLU() for _ in range(3)]).eval()
    m = PiscesLxFusedMoEDispatch(3, 2).eval()
    with pytest.raises(NotImplementedError, match="gradients"):
        m(x.requires_grad_(), w, idx, experts)
    x, w, idx = _inputs()
    with pytest.raises(NotImplementedError, match="gradients"):
        m(x, w.requires_grad_(), idx, experts)


def test_size_mismatch_raises_value_error():
    x, w, idx = _inputs()
    experts = nn.ModuleList([_SwiGLU() for _ in range(3)]).eval()
    m = PiscesLxFusedMoEDispatch(3, 2).eval()
    with pytest.raises(ValueError, match="assignments cannot come from"):
        m(x, w, idx.reshape(-1)[:-1], experts)
    with pytest.raises(ValueError, match="routing weights"):
        m(x, w[:-1], idx, experts)
