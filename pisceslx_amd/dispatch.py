"""PiscesLxFusedMoEDispatch for MI355X: the sort-based MoE dispatch operator.

Mirrors ``PiscesLxFusedMoEDispatch`` and ``PiscesLxFusedMoe.fused_moe_dispatch``
(opss/infer/fused_moe.py:32-143): same constructor, same ``forward(x_flat, routing_weights,
expert_indices, experts, collect_stats=False)`` contract, same ValueError for an index tensor
whose size does not match the token count (fused_moe.py:76-82). The work runs in libyvmoe
(``yvmoe_dispatch``): counts, offsets and the stable expert-sorted order on the device, the
grouped SwiGLU FFN of every (token, slot), the weighted combine — with no host
synchronization, where the reference copies the offsets to the host (fused_moe.py:96-97).

``experts`` is the packed routed-expert stack (:class:`pisceslx_amd.quant.PackedExperts`, any
weight format), or the reference's ``nn.ModuleList`` of SwiGLU experts (``gate_proj``,
``up_proj``, ``down_proj`` linears without bias), packed once to the activation dtype and
repacked when a weight changes.

Differences a caller can observe, all deliberate:
* the combine sums the slots of a token in fp32 in slot order and rounds once; the
  reference rounds each weighted product and each ``index_add_`` to the output dtype (on a
  GPU in an unordered atomic sequence), and with fp32 weights and bf16 activations its
  ``index_add_`` raises (source and destination dtypes differ), where this operator computes;
* the operator is an inference forward: in training mode (the module's or an expert's), or
  with inputs that require grad while autograd is on, it raises NotImplementedError instead of
  returning a detached output without the experts' dropout;
* an index outside ``[0, E)`` is never read through: those slots add nothing, and with
  ``check_indices`` (the default) the forward raises RuntimeError as the reference's bincount
  / module indexing does — that check reads one int from the device; set
  ``check_indices = False`` for a forward with no host synchronization.
"""
from __future__ import annotations

from typing import List, Optional, Sequence, Union

import torch
import torch.nn as nn

from . import _lib
from . import functional as yvf
from .quant import PackedExperts, pack_experts

ExpertsArg = Union[PackedExperts, Sequence[nn.Module]]


def _expert_linears(m: nn.Module):
    lins = []
    for name in ("gate_proj", "up_proj", "down_proj"):
        lin = getattr(m, name, None)
        if not isinstance(lin, nn.Linear):
            raise TypeError(f"expert {type(m).__name__} has no nn.Linear {name}: only SwiGLU "
                            "experts (YvSwiGLUExpert, model/moe/expert.py:475-489) are supported")
        if lin.bias is not None:
            raise NotImplementedError("SwiGLU experts with biases are not supported by the kernels")
        lins.append(lin)
    return lins


def packed_from_modules(experts: Sequence[nn.Module], dtype: torch.dtype, device) -> PackedExperts:
    """The routed-expert stack of a list of SwiGLU expert modules in the activation dtype
    (bf16 weights for bf16 activations, fp32 for fp32), cached on the list and repacked when
    any weight changes (its storage or its version counter)."""
    weights = [[lin.weight for lin in _expert_linears(m)] for m in experts]
    key = (dtype, str(device), tuple((w.data_ptr(), w._version) for ws in weights for w in ws))
    cached = getattr(experts, "_yvmoe_packed", None)
    if cached is not None and cached[0] == key:
        return cached[1]
    fmt = _lib.W_BF16 if dtype == torch.bfloat16 else _lib.W_F32
    with torch.no_grad():
        packed = pack_experts([tuple(w.detach().to(device) for w in ws) for ws in weights],
                              len(weights), fmt, device=device)
    try:
        experts._yvmoe_packed = (key, packed)
    except AttributeError:  # a plain tuple: no cache
        pass
    return packed


def _reject_training(module: nn.Module, x_flat: torch.Tensor, routing_weights: torch.Tensor,
                     experts: ExpertsArg) -> None:
    """The kernels are an inference forward: no autograd graph and no expert dropout
    (``YvSwiGLUExpert.forward`` applies dropout in training mode, model/moe/expert.py:484-489).
    A call that would need either raises instead of returning a detached output."""
    if module.training:
        raise NotImplementedError("PiscesLxFusedMoEDispatch on MI355X is an inference operator; "
                                  "call .eval()")
    if torch.is_grad_enabled() and (x_flat.requires_grad or routing_weights.requires_grad):
        raise NotImplementedError("PiscesLxFusedMoEDispatch on MI355X computes no gradients: run "
                                  "it under torch.no_grad() / inference_mode or pass tensors that "
                                  "do not require grad")
    if not isinstance(experts, PackedExperts):
        for m in experts:
            if m.training:
                raise NotImplementedError("expert modules in training mode (dropout active) are "
                                          "not supported; call .eval() on the experts")


class PiscesLxFusedMoEDispatch(nn.Module):
    """Sort-based MoE dispatch (opss/infer/fused_moe.py:32-123) on the MI355X kernels."""

    def __init__(self, num_experts: int, top_k: int) -> None:
        super().__init__()
        self.num_experts = num_experts
        self.top_k = top_k
        self.check_indices = True
        self._workspace: Optional[torch.Tensor] = None

    def forward(self, x_flat: torch.Tensor, routing_weights: torch.Tensor,
                expert_indices: torch.Tensor, experts: ExpertsArg, collect_stats: bool = False):
        _reject_training(self, x_flat, routing_weights, experts)
        num_tokens = x_flat.shape[0]
        hidden = x_flat.shape[-1]
        flat_indices = expert_indices.reshape(-1)
        num_assignments = flat_indices.numel()
        # the gate's own width is authoritative (fused_moe.py:72-82)
        per_token = expert_indices.shape[-1] if expert_indices.dim() > 1 else 1
        if num_assignments != num_tokens * per_token:
            raise ValueError(
                f"fused dispatch: {num_assignments} assignments cannot come from "
                f"{num_tokens} tokens with {per_token} experts each")
        if routing_weights.numel() != num_assignments:
            raise ValueError(f"fused dispatch: {routing_weights.numel()} routing weights for "
                             f"{num_assignments} assignments")
        dev = x_flat.device
        packed = experts if isinstance(experts, PackedExperts) else \
            packed_from_modules(experts, x_flat.dtype, dev)
        if num_assignments == 0:
            out = torch.zeros_like(x_flat)
            return (out, []) if collect_stats else out
        x2 = x_flat.reshape(num_tokens, hidden).contiguous()
        idx = flat_indices.reshape(num_tokens, per_token).to(torch.int64).contiguous()
        w = routing_weights.reshape(num_tokens, per_token)
        if w.dtype not in (torch.float32, torch.bfloat16):
            w = w.float()
        w = w.contiguous()
        need = yvf.dispatch_workspace_bytes(num_tokens, yvf._act(x2.dtype), per_token, packed)
        if self._workspace is None or self._workspace.numel() < need or self._workspace.device != dev:
            self._workspace = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
        out, counts, offsets, invalid, y = yvf.dispatch(x2, w, idx, packed,
                                                        want_expert_outputs=collect_stats,
                                                        workspace=self._workspace)
        if self.check_indices:
            bad = int(invalid.item())
            if bad:
                raise RuntimeError(f"fused dispatch: {bad} expert indices outside "
                                   f"[0, {packed.num_routed})")
        out = out.reshape(x_flat.shape)
        if collect_stats:
            # mean expert output of each active expert, in expert order (fused_moe.py:109-110)
            offs = offsets.tolist()
            stats: List[torch.Tensor] = [y[offs[e]:offs[e + 1]].mean(dim=0)
                                         for e in range(packed.num_routed) if offs[e + 1] > offs[e]]
            return out, stats
        return out


class PiscesLxFusedMoe:
    """Module-level operations of fused_moe (opss/infer/fused_moe.py:125-143)."""

    @staticmethod
    def fused_moe_dispatch(x_flat: torch.Tensor, routing_weights: torch.Tensor,
                           expert_indices: torch.Tensor, experts: ExpertsArg, num_experts: int,
                           top_k: int) -> torch.Tensor:
        # a functional call: the operator itself holds no training state (the experts' and the
        # inputs' are still checked)
        return PiscesLxFusedMoEDispatch(num_experts, top_k).eval()(x_flat, routing_weights,
                                                                  expert_indices, experts)
