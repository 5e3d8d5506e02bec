"""YvStableMoEGate for MI355X: the router of the Yv MoE layer.

Mirrors ``YvStableMoEGate`` (model/moe/gate.py:847-1247): same constructor arguments, same
parameter/buffer names (so a reference state_dict loads), same ``forward(x) -> (weights,
top_idx, loss)`` contract. The arithmetic runs in libyvmoe: the gate GEMM and the complexity
predictor on MFMA, then the routing kernels (softmax, top-k, double softmax, capacity trim,
renormalisation).

Inference only. Differences a caller can observe, all deliberate:
* the router computes in fp32 whatever the gate weight's dtype, so ``weights`` are fp32
  (the reference returns them in the logits' dtype, gate.py:1223);
* training-mode forwards (routing history, bias updates, noise, gate.py:1183-1190,
  :1206-1209, :1244-1245) raise NotImplementedError;
* a loaded module whose routing history makes the reference add random noise
  (balance_ratio < 0.7, gate.py:1206) raises NotImplementedError; the deterministic load
  adjustment 0.1 * (predicted - recent) (gate.py:1203-1204) is supported;
* ``enable_cognitive_density`` builds no modules: the reference forward never calls them.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn as nn

from . import _lib
from . import functional as yvf
from .quant import pack_router


class YvStableMoEGate(nn.Module):
    def __init__(self, hidden_size, num_experts, top_k=2, device=None, dtype=None,
                 capacity_factor=1.0, min_capacity=4, prediction_horizon=10,
                 fixed_shape_mode=False, enable_dynamic_capacity=True,
                 enable_cognitive_density=False):
        super().__init__()
        if not 1 <= num_experts <= _lib.MAX_EXPERTS:
            raise ValueError(f"num_experts={num_experts} outside [1, {_lib.MAX_EXPERTS}]")
        self.gate = nn.Linear(hidden_size, num_experts, bias=False, device=device, dtype=dtype)
        self.top_k = top_k
        self.num_experts = num_experts
        self.capacity_factor = capacity_factor
        self.min_capacity = min_capacity
        self.prediction_horizon = prediction_horizon
        self.fixed_shape_mode = fixed_shape_mode
        self.enable_dynamic_capacity = enable_dynamic_capacity
        self.enable_cognitive_density = enable_cognitive_density
        if enable_dynamic_capacity:
            # built without device/dtype in the reference (gate.py:930-936): fp32
            self.complexity_predictor = nn.Sequential(
                nn.Linear(hidden_size, 64), nn.ReLU(), nn.Linear(64, 1), nn.Sigmoid()).to(device)
        self.register_buffer("routing_history", torch.zeros(100, num_experts, device=device))
        self.register_buffer("history_ptr", torch.tensor(0, device=device))
        self.load_predictor = nn.LSTM(input_size=num_experts, hidden_size=64, num_layers=2,
                                      batch_first=True, dropout=0.1).to(device)
        self.predictor_head = nn.Linear(64, num_experts * prediction_horizon).to(device)
        self.register_buffer("expert_load_buffer", torch.zeros(50, num_experts, device=device))
        self.register_buffer("load_buffer_ptr", torch.tensor(0, device=device))
        self.register_buffer("expert_bias", torch.zeros(num_experts, device=device))
        self.bias_update_rate = 0.05
        self.bias_update_freq = 50
        self.register_buffer("bias_update_counter", torch.tensor(0, device=device))
        self.register_buffer("total_routing_count", torch.tensor(0.0, device=device))
        self._is_checkpointing = False
        self._packed = None
        self._packed_key = None

    # ------------------------------------------------------------ host-side state
    def _load_adjustment(self) -> Optional[torch.Tensor]:
        """0.1 * (predicted - recent usage) of gate.py:1192-1209, or None when inactive.

        Computed on the host side from the routing-history buffers, which an inference forward
        never changes, so the result is cached on the buffers' versions (no device sync per call).
        """
        key = tuple((b.data_ptr(), b._version) for b in (
            self.history_ptr, self.load_buffer_ptr, self.routing_history, self.expert_load_buffer))
        if getattr(self, "_adj_key", None) == key:
            return self._adj
        self._adj = self._compute_load_adjustment()
        self._adj_key = key
        return self._adj

    def _compute_load_adjustment(self) -> Optional[torch.Tensor]:
        hp = int(self.history_ptr.item())
        if hp <= 0:
            return None
        E = self.num_experts
        lp = int(self.load_buffer_ptr.item())
        if lp < 10:
            predicted = torch.ones(E, device=self.routing_history.device) / E
        else:
            with torch.no_grad():
                hist = self.expert_load_buffer[:lp].unsqueeze(0).float()
                out, _ = self.load_predictor(hist)
                pred = self.predictor_head(out[:, -1, :])
            predicted = torch.softmax(pred.view(E, self.prediction_horizon).mean(dim=1), dim=0)
        recent = self.routing_history[:hp].mean(0).float()
        entropy = -torch.sum(recent * torch.log(recent.clamp(min=1e-8)))
        ratio = float(entropy) / max(1e-8, math.log(E))
        if ratio < 0.7:
            raise NotImplementedError(
                "YvStableMoEGate state adds random routing noise (balance_ratio "
                f"{ratio:.3f} < 0.7, gate.py:1206); the inference kernels do not reproduce it")
        return (0.1 * (predicted.float() - recent)).contiguous()

    def router_state(self, act: int) -> yvf.RouterState:
        """Packed device tensors for the router GEMM (repacked when parameters change)."""
        w = self.gate.weight
        pred = getattr(self, "complexity_predictor", None)
        key = (act, w.data_ptr(), w._version,
               None if pred is None else tuple((p.data_ptr(), p._version) for p in pred.parameters()))
        if self._packed is None or self._packed_key != key:
            w1 = pred[0].weight.detach() if pred is not None else None
            b1 = pred[0].bias.detach().float().contiguous() if pred is not None else None
            w2 = pred[2].weight.detach().float().reshape(-1).contiguous() if pred is not None else None
            b2 = pred[2].bias.detach().float().reshape(-1).contiguous() if pred is not None else None
            self._packed = (pack_router(w.detach(), w1, act), b1, w2, b2)
            self._packed_key = key
        w_router, b1, w2, b2 = self._packed
        if self.fixed_shape_mode:
            bias = self.expert_bias.float().contiguous()
        else:
            bias = self._load_adjustment()
        return yvf.RouterState(self.num_experts, self.gate.in_features, min(self.top_k, self.num_experts),
                               bool(self.fixed_shape_mode), bool(self.enable_dynamic_capacity),
                               int(self.min_capacity), float(self.capacity_factor), w_router, b1, w2,
                               b2, bias)

    def _check_inference(self):
        if self.training:
            raise NotImplementedError(
                "the MI355X YvStableMoEGate is an inference forward; call .eval() first")

    # ------------------------------------------------------------ forward
    def forward(self, x: torch.Tensor):
        """(weights [N,k] fp32, top_idx [N,k] int64, loss) for x [B, S, H] (gate.py:1122)."""
        self._check_inference()
        B, S, H = x.shape
        x2d = x.reshape(-1, H).contiguous()
        act = yvf._act(x2d.dtype)
        st = self.router_state(act)
        logits = yvf.router_logits(x2d, st)
        routing = yvf.route(logits, st, predictor=True)
        return routing.weights, routing.indices, torch.tensor(0.0, device=x.device)

    def route_logits(self, logits: torch.Tensor, capacity: Optional[int] = None) -> yvf.Routing:
        """Routing of given fp32 logits [N, E] (no predictor: pass ``capacity`` in dynamic mode)."""
        self._check_inference()
        st = self.router_state(_lib.ACT_F32)
        cap = -1 if capacity is None else int(capacity)
        return yvf.route(logits.float().contiguous(), st, predictor=False, capacity_override=cap)
