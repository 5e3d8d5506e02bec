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
import torch.nn.functional as F

from . import _lib
from . import functional as yvf
from .quant import block_matrix, pack_router


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


class _YvDGEncoder(nn.Module):
    """Parameters of YvDGEncoder (model/moe/hicl_router.py:50-85): dg_proj and dg_bias; the
    relu / top-k / L2 normalisation run in the gate kernel."""

    def __init__(self, hidden_size, expansion_factor=4, sparsity_k=32, device=None, dtype=None):
        super().__init__()
        self.hidden_size = hidden_size
        self.dg_dim = hidden_size * expansion_factor
        self.sparsity_k = sparsity_k
        self.dg_proj = nn.Linear(hidden_size, self.dg_dim, bias=False, device=device, dtype=dtype)
        self.register_buffer("dg_bias", torch.zeros(self.dg_dim, device=device, dtype=dtype))


class YvMoEGate(nn.Module):
    """YvMoEGate for MI355X: the router the reference's MoE layers build (layer.py:754-777).

    Mirrors ``YvMoEGate`` (model/moe/gate.py:140-451): same constructor arguments, parameter
    and buffer names, ``forward(x, modal_id=None) -> (top_scores, top_idx, loss)``. Inference
    only: the standard gate plus the four auxiliary heads (HiCL, Graph-of-Tokens cluster
    projection, SoftMoE, Expert-Oriented), modal affinity, expert bias and temperature run in
    ``yvmoe_moegate_logits``; the softmax / top-k / softmax of the k scores in ``yvmoe_route``
    (fixed mode); the PathMoE stage cache (gate.py:418-431) is kept on the module.

    Differences a caller can observe, all deliberate:
    * logits are computed in fp32 whatever the parameter dtype (the reference's chain runs in
      the parameter dtype); ``top_scores`` are the fp32 softmax cast to x's dtype, as the
      reference casts them (gate.py:416);
    * ``got_graph_builder`` (whose output the reference computes under no_grad and never
      uses, gate.py:345-346) and ``importance_proj`` (whose tiers the top-k never reads,
      gate.py:396-402) are not built; their keys in a reference state_dict are skipped on load;
    * training-mode forwards raise NotImplementedError;
    * after ``prune_routing_heads`` the pruned heads are left out of the logits, as
      ``_should_compute_aux_head`` intends (gate.py:263-276); the reference's forward instead
      raises AttributeError, since it reads the deleted ``sparse_gate_*`` before that check
      (gate.py:331-333).
    """

    HEAD_NAMES = (("hicl", _lib.HEAD_HICL), ("got", _lib.HEAD_GOT),
                  ("soft_moe", _lib.HEAD_SOFT), ("expert_orient", _lib.HEAD_EO))
    _SKIPPED_PREFIXES = ("got_graph_builder.", "importance_proj.")

    def __init__(self, hidden_size, num_experts, top_k=2, device=None, dtype=None,
                 load_balance_alpha=0.01, noise_std=0.1, enable_cognitive_density=False,
                 expert_capacity_limit=1.2, dynamic_top_k_min=1, dynamic_top_k_max=3,
                 load_balance_threshold=0.15, cfg=None):
        super().__init__()
        if not 1 <= num_experts <= _lib.MAX_EXPERTS:
            raise ValueError(f"num_experts={num_experts} outside [1, {_lib.MAX_EXPERTS}]")
        c = lambda name, default: getattr(cfg, name, default) if cfg is not None else default
        f = dict(device=device, dtype=dtype)
        self.top_k = top_k
        self.num_experts = num_experts
        self.hidden_size = hidden_size
        self.load_balance_alpha = load_balance_alpha
        self.noise_std = max(noise_std, 0.2)
        self.enable_cognitive_density = enable_cognitive_density
        self.expert_capacity_limit = expert_capacity_limit
        self.dynamic_top_k_min = dynamic_top_k_min
        self.dynamic_top_k_max = dynamic_top_k_max
        self.load_balance_threshold = load_balance_threshold
        self.z_loss_alpha = c("moe_z_loss_alpha", 1e-4)
        self.random_to_gradient_steps = c("moe_random_to_gradient_steps", 2000)
        self.attention_mamba_temp = c("moe_attention_mamba_temp", 0.3)
        self.min_temperature = c("moe_temperature_min", 1.5)
        self.register_buffer("expert_usage_count", torch.zeros(num_experts, **f))
        self.register_buffer("temperature", torch.tensor(c("moe_routing_temperature", 3.0), **f))
        self.register_buffer("total_routing_count", torch.tensor(0.0, **f))
        self.register_buffer("expert_temperature_max", torch.tensor(c("moe_temperature_max", 5.0), **f))
        self.register_buffer("expert_bias", torch.zeros(num_experts, **f))
        self.register_buffer("bias_update_counter", torch.tensor(0, **f))
        self._is_checkpointing = False
        self.gate = nn.Linear(hidden_size, num_experts, bias=False, **f)
        # HiCL
        self.hicl_dg_dim = hidden_size * 4
        self.hicl_dg_encoder = _YvDGEncoder(hidden_size, 4, 32, **f)
        self.hicl_prototypes = nn.Parameter(torch.randn(num_experts, self.hicl_dg_dim, **f) * 0.02)
        self.w_hicl = nn.Parameter(torch.tensor(0.1, **f))
        # Graph-of-Tokens: only the cluster projection reaches the logits
        self.got_cluster_proj = nn.Linear(hidden_size, num_experts, bias=False, **f)
        self.w_got = nn.Parameter(torch.tensor(0.05, **f))
        # SoftMoE
        self.soft_moe_temperature = c("soft_moe_temperature", 1.0)
        self.gate_k = nn.Linear(hidden_size, num_experts, bias=False, **f)
        self.gate_v = nn.Linear(hidden_size, num_experts, bias=False, **f)
        self.register_buffer("soft_moe_budget", torch.tensor(float(c("soft_moe_mean_k", top_k)), **f))
        self.w_soft = nn.Parameter(torch.tensor(0.05, **f))
        # Expert-Oriented
        D = max(64, hidden_size // 64)
        self.expert_embeddings = nn.Parameter(torch.randn(num_experts, D, **f))
        self.input_encoder = nn.Sequential(nn.Linear(hidden_size, D, bias=False, **f), nn.SiLU(),
                                           nn.Linear(D, D, bias=False, **f))
        self.expert_capability_encoder = nn.Sequential(nn.Linear(D, D, bias=False, **f), nn.SiLU(),
                                                       nn.Linear(D, D, bias=False, **f))
        self.w_expert_orient = nn.Parameter(torch.tensor(0.05, **f))
        # Modal-aware affinity (n_modalities 7 without a cfg, as gate.py:247)
        self.n_modalities = c("n_modalities", 5) if cfg is not None else 7
        self.expert_modal_affinity = nn.Parameter(torch.zeros(num_experts, self.n_modalities, **f))
        self.affinity_alpha = 1.0
        # PathMoE cache
        self._path_moe_stage_size = c("path_moe_stage_size", 4)
        self._path_moe_layer_idx = 0
        self._path_moe_cache = None
        self._path_moe_signature = None
        self.sparse_gate_hicl = nn.Parameter(torch.tensor(5.0, **f))
        self.sparse_gate_got = nn.Parameter(torch.tensor(5.0, **f))
        self.sparse_gate_soft_moe = nn.Parameter(torch.tensor(5.0, **f))
        self.sparse_gate_expert_orient = nn.Parameter(torch.tensor(5.0, **f))
        self._pruned_heads: set = set()
        self._state = None
        self._state_key = None
        self._register_load_state_dict_pre_hook(self._skip_unbuilt_keys)
        self.last_routing: Optional[yvf.Routing] = None
        self._workspace: Optional[torch.Tensor] = None
        self._tlist_key = None
        self._tlist_probe = ()

    def _skip_unbuilt_keys(self, state_dict, prefix, *args):
        for k in [k for k in state_dict if k.startswith(tuple(prefix + p for p in self._SKIPPED_PREFIXES))]:
            del state_dict[k]

    # ------------------------------------------------------------ host-side state
    def _host_constants(self, seq_len: int):
        """Effective temperature (gate.py:297-308) and the capacity term (gate.py:586-591),
        both from buffers, evaluated in the buffers' dtype as the reference does."""
        t = self.temperature.detach().cpu()
        if seq_len >= 8192:
            t = t * self.attention_mamba_temp
        hi = self.expert_temperature_max.detach().cpu().to(t.dtype)
        t = torch.max(torch.min(t, hi), torch.tensor(0.1, dtype=t.dtype))
        cap = 0.0
        total = self.total_routing_count.detach().cpu()
        if float(total) > 0:
            usage = self.expert_usage_count.detach().cpu() / total
            cap = float(0.005 * torch.sum(torch.relu(usage - self.expert_capacity_limit) ** 2))
        return float(t), cap

    def gate_state(self, act: int, seq_len: int) -> yvf.MoEGateState:
        """Regrouped device tensors for yvmoe_moegate_logits (rebuilt when a parameter,
        buffer or the pruned set changes)."""
        tensors = self._tensor_list()
        key = (act, seq_len >= 8192, tuple(sorted(self._pruned_heads)),
               tuple((t.data_ptr(), t._version) for t in tensors))
        if self._state is not None and self._state_key == key:
            return self._state
        wdt = torch.bfloat16 if act == _lib.ACT_BF16 else torch.float32
        E, H = self.num_experts, self.hidden_size
        D = self.expert_embeddings.shape[1]
        heads = 0
        for name, bit in self.HEAD_NAMES:
            if name not in self._pruned_heads:
                heads |= bit
        enc = self.hicl_dg_encoder
        with torch.no_grad():
            dev = self.gate.weight.device
            # [dg_proj (with HiCL); gate; got_cluster_proj; gate_k; gate_v; input_encoder.0; 0]
            dg = enc.dg_dim if heads & _lib.HEAD_HICL else 0
            rh = (4 * E + D + 255) // 256 * 256
            w_proj = torch.zeros(dg + rh, H, dtype=wdt, device=dev)
            if dg:
                w_proj[:dg] = enc.dg_proj.weight
            w_proj[dg:dg + E] = self.gate.weight
            w_proj[dg + E:dg + 2 * E] = self.got_cluster_proj.weight
            w_proj[dg + 2 * E:dg + 3 * E] = self.gate_k.weight
            w_proj[dg + 3 * E:dg + 4 * E] = self.gate_v.weight
            w_proj[dg + 4 * E:dg + 4 * E + D] = self.input_encoder[0].weight
            if act == _lib.ACT_BF16:
                w_proj = block_matrix(w_proj, _lib.W_BF16)  # the GEMM kernels' blocked order
            dg_bias = enc.dg_bias.detach().float().contiguous()
            proto_t = self.hicl_prototypes.detach().float().t().contiguous()
            # Expert-Oriented: silu(enc0 x) · enc2ᵀ · eeᵀ with ee = cap2(silu(cap0(emb))), a
            # constant of the weights; both linear maps after the SiLU fold into one [D, E]
            cap0 = self.expert_capability_encoder[0].weight.detach().double()
            cap2 = self.expert_capability_encoder[2].weight.detach().double()
            ee = F.silu(self.expert_embeddings.detach().double() @ cap0.t()) @ cap2.t()
            eo_mat = (self.input_encoder[2].weight.detach().double().t() @ ee.t()).float().contiguous()
            modal = self.expert_modal_affinity.detach().float().contiguous()
            ebias = self.expert_bias.detach().float().contiguous()
        temp, cap_loss = self._host_constants(seq_len)
        pdt = self.gate.weight.dtype
        soft_eps = max(1e-8, torch.finfo(pdt).eps * 10) if pdt in (torch.float16, torch.bfloat16) else 1e-8
        scalar = lambda name: (float(getattr(self, name).detach().float().cpu())
                               if hasattr(self, name) else 0.0)
        self._state = yvf.MoEGateState(
            E, H, D, enc.dg_dim, min(enc.sparsity_k, enc.dg_dim), self.n_modalities, heads,
            w_proj, dg_bias, proto_t, eo_mat, modal, ebias,
            scalar("w_hicl"), scalar("w_got"), scalar("w_soft"),
            scalar("w_expert_orient"), float(self.soft_moe_temperature), temp, soft_eps,
            float(self.load_balance_alpha), float(self.z_loss_alpha),
            scalar("soft_moe_budget"), cap_loss)
        self._state_key = key
        return self._state

    def _tensor_list(self):
        """Parameters and buffers, listed once per module structure (pruning or device moves
        change the objects, which changes the key)."""
        ids = (len(self._parameters), len(self._buffers), tuple(sorted(self._pruned_heads)))
        if getattr(self, "_tlist_key", None) != ids or any(
                t is not p for t, p in zip(self._tlist_probe, (self.gate.weight, self.temperature))):
            self._tlist = list(self.parameters()) + list(self.buffers())
            self._tlist_probe = (self.gate.weight, self.temperature)
            self._tlist_key = ids
        return self._tlist

    def fixed_router_state(self) -> yvf.RouterState:
        """The fixed-mode routing (softmax, top-k, softmax of the k scores) on the gate logits."""
        return yvf.RouterState(self.num_experts, self.hidden_size, min(self.top_k, self.num_experts),
                               True, False, 0, 1.0, None, None, None, None, None)

    def _modal_ids(self, modal_id: torch.Tensor, B: int, S: int, device) -> torch.Tensor:
        """modal_id reshaped as gate.py:369-374 does, to int32 [B*S], range-checked."""
        m = modal_id
        if tuple(m.shape) != (B, S):
            m = m.reshape(B, 1).expand(B, S) if m.numel() == B else m.reshape(B, S)
        m = m.reshape(-1).to(device=device, dtype=torch.int32).contiguous()
        if m.numel() and (int(m.min()) < -self.n_modalities or int(m.max()) >= self.n_modalities):
            raise IndexError(f"modal_id outside [-{self.n_modalities}, {self.n_modalities})")
        return torch.where(m < 0, m + self.n_modalities, m)

    # ------------------------------------------------------------ forward
    def forward(self, x: torch.Tensor, modal_id: Optional[torch.Tensor] = None):
        if self.training:
            raise NotImplementedError("the MI355X YvMoEGate is an inference forward; call .eval() first")
        B, S, H = x.shape
        x2d = x.reshape(-1, H).contiguous()
        act = yvf._act(x2d.dtype)
        st = self.gate_state(act, S)
        mid = None if modal_id is None else self._modal_ids(modal_id, B, S, x.device)
        N = x2d.shape[0]
        cached = self.path_moe_begin(N)
        ws = self._workspace if getattr(self, "_workspace", None) is not None and \
            self._workspace.device == x.device else None
        logits, loss, fresh, ws = yvf.moegate_forward(x2d, st, min(self.top_k, self.num_experts),
                                                      mid, workspace=ws)
        self._workspace = ws
        routing = cached[1] if cached is not None else fresh
        self.path_moe_end(None if cached is not None else (logits, fresh))
        self.last_routing = routing
        self.last_logits = logits
        self._last_loss_f32 = loss
        return routing.weights.to(x.dtype), routing.indices, loss.reshape(()).to(x.dtype)

    # PathMoE (gate.py:418-431): one routing shared by a stage of calls with the same token
    # count; the later calls of a stage keep it (their own logits still set the loss).
    def path_moe_begin(self, n_tokens: int):
        """Stage bookkeeping before a forward: the cached (logits, routing) to reuse, or None."""
        if self._path_moe_stage_size <= 1:
            return None
        sig = (n_tokens, self.training)
        if sig != self._path_moe_signature:
            self._path_moe_layer_idx = 0
            self._path_moe_cache = None
            self._path_moe_signature = sig
        if self._path_moe_layer_idx != 0 and self._path_moe_cache is not None:
            return self._path_moe_cache
        return None

    def path_moe_end(self, fresh) -> None:
        """After a forward: cache this call's (logits, routing) when it routed afresh."""
        if self._path_moe_stage_size <= 1:
            return
        if fresh is not None:
            self._path_moe_cache = fresh
        self._path_moe_layer_idx = (self._path_moe_layer_idx + 1) % self._path_moe_stage_size

    def prune_routing_heads(self, prune_threshold: float = 0.05) -> None:
        """Drop auxiliary heads whose sparse gate sigmoid is below the threshold (gate.py:466-489)."""
        for name, attr in (("hicl", "sparse_gate_hicl"), ("got", "sparse_gate_got"),
                           ("soft_moe", "sparse_gate_soft_moe"),
                           ("expert_orient", "sparse_gate_expert_orient")):
            p = getattr(self, attr, None)
            if p is not None and float(torch.sigmoid(p.detach().float())) < prune_threshold:
                self._pruned_heads.add(name)
                delattr(self, attr)
                if hasattr(self, f"w_{name}"):
                    delattr(self, f"w_{name}")
