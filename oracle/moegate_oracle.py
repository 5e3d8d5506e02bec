"""CPU oracle of the YvMoEGate inference forward — TEST INFRASTRUCTURE ONLY.

Only tests/ may import this module (as the checker of the GPU path); the product package
``pisceslx_amd`` never imports it.

Restates ``YvMoEGate.forward`` in eval mode, model/moe/gate.py:310-451, in float64 from the
module's parameters (a state dict with the reference's keys):

* step 2 — ``logits = gate(x)`` plus the four auxiliary heads, each scaled by its weight
  ``w_*`` times ``straight_through_gate(sparse_gate_*)``, which is exactly 1.0
  (model/utils/safety.py:37-49):
  HiCL (gate.py:335-340; ``YvDGEncoder`` model/moe/hicl_router.py:70-85: relu(x Wdgᵀ + b),
  the top-32 entries kept, L2-normalised with eps 1e-12, times the prototypes); Graph-of-Tokens
  (gate.py:343-348: only ``got_cluster_proj(x)`` reaches the logits, the token graph built under
  no_grad is unused); SoftMoE (gate.py:351-358: sigmoid((k - median_e(k)) / T) · softmax(v),
  divided by max(sum, eps(dtype))); Expert-Oriented (gate.py:361-366:
  ``input_encoder(x) · expert_capability_encoder(expert_embeddings)ᵀ``);
* step 3 — modal affinity bias ``expert_modal_affinity[:, modal_id]`` (gate.py:369-376);
* step 4 — ``+ expert_bias``;
* step 7 — temperature: ``logits / clamp(temperature · (0.3 if seq_len >= 8192 else 1), 0.1,
  expert_temperature_max)`` (gate.py:297-308), evaluated as the reference does, in the
  buffers' dtype (``effective_temperature``);
* step 8/10 — ``softmax``, ``topk``, softmax of the k scores (gate.py:393, :414-416);
* step 13 — the eval loss: load balance ``alpha · Σ_e (mean_n scores - 1/E)²`` plus the
  capacity penalty from the usage buffers (gate.py:556-593), z-loss
  ``z_alpha · mean(logits²)`` on the temperature-scaled logits (gate.py:595-610), and the
  SoftMoE budget term ``0.01 · (mean_n Σ_e soft - budget)²`` (gate.py:440-444).

Pruned heads (``heads``, gate.py:263-276) are left out of the sum, and without SoftMoE the
budget term is 0 (gate.py:440-444).

The PathMoE cache (gate.py:418-431) is module state, not arithmetic; the module's tests cover it.
Ties in torch.topk over the DG activations are not specified by torch; the restatement keeps
the lower index, which only matters for exactly equal activations at the 32nd place.

Parity status: pinned by tests/test_oracle_moegate.py (closed forms with heads switched off,
brute-force top-k and lower median, sparse-vector norms, SoftMoE normalisation, temperature
rules, loss terms on hand-built inputs).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional

import numpy as np
import torch
import torch.nn.functional as F


@dataclass
class MoEGateParams:
    """float64 view of a YvMoEGate's parameters and eval constants."""
    gate: torch.Tensor            # [E, H]
    dg_proj: torch.Tensor         # [4H, H]
    dg_bias: torch.Tensor         # [4H]
    prototypes: torch.Tensor      # [E, 4H]
    got_proj: torch.Tensor        # [E, H]
    gate_k: torch.Tensor          # [E, H]
    gate_v: torch.Tensor          # [E, H]
    enc0: torch.Tensor            # [D, H]  input_encoder.0
    enc2: torch.Tensor            # [D, D]  input_encoder.2
    cap0: torch.Tensor            # [D, D]  expert_capability_encoder.0
    cap2: torch.Tensor            # [D, D]  expert_capability_encoder.2
    expert_embeddings: torch.Tensor  # [E, D]
    modal_affinity: torch.Tensor  # [E, M]
    expert_bias: torch.Tensor     # [E]
    w_hicl: float
    w_got: float
    w_soft: float
    w_eo: float
    temperature: float
    temperature_max: float
    soft_temperature: float = 1.0
    soft_budget: float = 2.0
    sparsity_k: int = 32
    load_balance_alpha: float = 0.01
    z_loss_alpha: float = 1e-4
    capacity_limit: float = 1.2
    usage_count: Optional[torch.Tensor] = None   # [E]
    total_routing_count: float = 0.0
    eps: float = 1e-8                            # YvNumericalGuard.get_eps(dtype)
    temp_dtype: torch.dtype = torch.float32      # dtype of the temperature buffers
    heads: frozenset = frozenset(("hicl", "got", "soft_moe", "expert_orient"))


def params_from_state_dict(sd: Dict[str, torch.Tensor], dtype: torch.dtype,
                           soft_temperature: float = 1.0, heads=None) -> MoEGateParams:
    """From a YvMoEGate state dict (the reference's keys); weights of pruned heads may be
    missing (prune_routing_heads deletes w_hicl / w_got, gate.py:484-489)."""
    d = lambda k: sd[k].detach().double().cpu()
    s = lambda k: float(sd[k].detach().double().cpu()) if k in sd else 0.0
    eps = 1e-8
    if dtype in (torch.float16, torch.bfloat16):
        eps = max(1e-8, torch.finfo(dtype).eps * 10)
    return MoEGateParams(
        gate=d("gate.weight"), dg_proj=d("hicl_dg_encoder.dg_proj.weight"),
        dg_bias=d("hicl_dg_encoder.dg_bias"), prototypes=d("hicl_prototypes"),
        got_proj=d("got_cluster_proj.weight"), gate_k=d("gate_k.weight"), gate_v=d("gate_v.weight"),
        enc0=d("input_encoder.0.weight"), enc2=d("input_encoder.2.weight"),
        cap0=d("expert_capability_encoder.0.weight"), cap2=d("expert_capability_encoder.2.weight"),
        expert_embeddings=d("expert_embeddings"), modal_affinity=d("expert_modal_affinity"),
        expert_bias=d("expert_bias"), w_hicl=s("w_hicl"), w_got=s("w_got"), w_soft=s("w_soft"),
        w_eo=s("w_expert_orient"), temperature=s("temperature"),
        temperature_max=s("expert_temperature_max"), soft_temperature=soft_temperature,
        soft_budget=s("soft_moe_budget"), usage_count=d("expert_usage_count"),
        total_routing_count=s("total_routing_count"), eps=eps, temp_dtype=sd["temperature"].dtype,
        **({} if heads is None else {"heads": frozenset(heads)}))


def effective_temperature(temperature: float, temperature_max: float, seq_len: int,
                          dtype: torch.dtype = torch.float32) -> float:
    """_safe_temperature's divisor (gate.py:297-308) computed in the buffers' dtype: the
    0.3 factor for seq_len >= 8192, then YvNumericalGuard.safe_clamp with a tensor upper bound
    (model/utils/safety.py:70-74: max(min(t, high), low))."""
    t = torch.tensor(temperature, dtype=dtype)
    if seq_len >= 8192:
        t = t * 0.3
    hi = torch.tensor(temperature_max, dtype=dtype)
    return float(torch.max(torch.min(t, hi), torch.tensor(0.1, dtype=dtype)))


def topk_lower_index(v: torch.Tensor, k: int):
    """Top-k values of each row, ties by lower index (stable descending sort)."""
    order = torch.from_numpy(np.argsort(-v.numpy(), axis=-1, kind="stable"))[:, :k]
    return torch.gather(v, 1, order), order


def lower_median(v: torch.Tensor) -> torch.Tensor:
    """torch.median along the last dim: the lower of the two middle values for even sizes."""
    s = torch.sort(v, dim=-1).values
    return s[:, (v.shape[-1] - 1) // 2]


def dg_sparse(x: torch.Tensor, p: MoEGateParams) -> torch.Tensor:
    """YvDGEncoder.forward: relu(x Wᵀ + b), top-k kept, L2-normalised (eps 1e-12)."""
    dg = torch.relu(x @ p.dg_proj.t() + p.dg_bias)
    k = min(p.sparsity_k, dg.shape[-1])
    vals, idx = topk_lower_index(dg, k)
    sparse = torch.zeros_like(dg).scatter_(1, idx, vals)
    return F.normalize(sparse, p=2, dim=-1, eps=1e-12)


def head_logits(x: torch.Tensor, p: MoEGateParams) -> Dict[str, torch.Tensor]:
    """The pieces of step 2 (float64), before the weights w_*."""
    hicl = dg_sparse(x, p) @ p.prototypes.t()
    got = x @ p.got_proj.t()
    soft = soft_weights(x, p)
    ie = F.silu(x @ p.enc0.t()) @ p.enc2.t()
    ee = F.silu(p.expert_embeddings @ p.cap0.t()) @ p.cap2.t()
    return {"gate": x @ p.gate.t(), "hicl": hicl, "got": got, "soft": soft, "eo": ie @ ee.t()}


def gate_loss(logits: torch.Tensor, soft: Optional[torch.Tensor], p: MoEGateParams) -> float:
    """The eval loss (gate.py:433-444, :556-610) of a batch's final logits [N, E] (float64)
    and, with the SoftMoE head on, its SoftMoE weights [N, E]: load balance over the mean
    scores plus the capacity term, z-loss, SoftMoE budget."""
    E = logits.shape[-1]
    scores = torch.softmax(logits, dim=-1)
    lb = p.load_balance_alpha * torch.sum((scores.mean(dim=0) - 1.0 / E) ** 2)
    if p.total_routing_count > 0:
        usage = p.usage_count / p.total_routing_count
        lb = lb + 0.005 * torch.sum(torch.relu(usage - p.capacity_limit) ** 2)
    z = p.z_loss_alpha * torch.mean(logits ** 2)
    budget = 0.0
    if "soft_moe" in p.heads:
        budget = 0.01 * (soft.sum(dim=-1).mean() - p.soft_budget) ** 2
    return float(lb + z + budget)


def soft_weights(x: torch.Tensor, p: MoEGateParams) -> torch.Tensor:
    """SoftMoE weights [N, E] of x [N, H] (float64), as head_logits computes them."""
    lk, lv = x @ p.gate_k.t(), x @ p.gate_v.t()
    sw = torch.sigmoid((lk - lower_median(lk)[:, None]) / p.soft_temperature)
    soft = sw * torch.softmax(lv, dim=-1)
    return soft / soft.sum(dim=-1, keepdim=True).clamp(min=p.eps)


def moegate_forward(x3d: torch.Tensor, p: MoEGateParams, k: int,
                    modal_id: Optional[torch.Tensor] = None,
                    seq_len: Optional[int] = None) -> Dict[str, object]:
    """Eval forward of x [B, S, H]: final logits (float64), scores, top-k weights / indices
    (from the float64 scores), and the loss terms. ``seq_len`` overrides S in the temperature
    rule (x then holds sampled tokens of longer sequences; the loss is over the given tokens)."""
    B, S, H = x3d.shape
    x = x3d.reshape(-1, H).double()
    E = p.gate.shape[0]
    h = head_logits(x, p)
    logits = h["gate"]
    for name, key, wt in (("hicl", "hicl", p.w_hicl), ("got", "got", p.w_got),
                          ("soft_moe", "soft", p.w_soft), ("expert_orient", "eo", p.w_eo)):
        if name in p.heads:
            logits = logits + wt * h[key]
    if modal_id is not None:
        m = modal_id
        if tuple(m.shape) != (B, S):
            m = m.reshape(B, 1).expand(B, S) if m.numel() == B else m.reshape(B, S)
        logits = logits + p.modal_affinity[:, m.reshape(-1).long()].t()
    logits = logits + p.expert_bias
    eff = effective_temperature(p.temperature, p.temperature_max, S if seq_len is None else seq_len,
                                p.temp_dtype)
    logits = logits / eff
    scores = torch.softmax(logits, dim=-1)
    kk = min(k, E)
    ts, idx = topk_lower_index(scores, kk)
    w = torch.softmax(ts, dim=-1)
    return {"logits": logits, "scores": scores, "weights": w, "indices": idx,
            "loss": gate_loss(logits, h["soft"], p), "heads": h, "temperature": eff}
