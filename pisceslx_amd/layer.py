"""Yv MoE layer forward for MI355X — drop-in for YvDynamicMoELayer / YvDeepSeekMoELayer.

Reference: model/moe/layer.py:519-963 (YvDynamicMoELayer) and :967-1396
(YvDeepSeekMoELayer). The router is what the reference's ``_build_router`` builds, YvMoEGate
(layer.py:754-777), by default (``router="moegate"``); ``router="stable"`` swaps in
YvStableMoEGate, the gate the reference's YvMoELayer builds (model/moe/gate.py:1498-1510).

``forward(x, subconscious_hints=None, modal_id=None) -> (out, loss)`` keeps the reference
signature; ``subconscious_hints`` is accepted and ignored, ``modal_id`` goes to YvMoEGate
(layer.py:903-909; YvStableMoEGate takes none). The loss is YvMoEGate's routing loss (0 with
YvStableMoEGate, whose inference forward has none). The stateful UltraMem skip residual
(layer.py:739-753) is kept: when shared experts exist, 0.1 * the previous call's shared
output is added if the shapes agree, and the buffer is replaced by this call's shared output.

The experts are stored stacked and packed (int8 / int4 g128 / fp8 128x128 / bf16 / fp32),
routed experts first, then the shared experts; ``load_reference_state_dict`` accepts the
reference keys ``experts.{e}.{gate,up,down}_proj.weight``,
``shared_experts.{s}.expert.{gate,up,down}_proj.weight``, ``shared_expert_weight`` and
``router.*``. The whole forward is one libyvmoe call on the current stream.
"""
from __future__ import annotations

import math
from typing import Any, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from . import functional as yvf
from .gate import YvMoEGate, YvStableMoEGate
from .quant import ExpertPacker, FORMAT_BY_NAME, FORMAT_NAMES, PackedExperts


def _kaiming_uniform(out_f: int, in_f: int, generator=None, device=None) -> torch.Tensor:
    # nn.init.kaiming_uniform_(a=sqrt(5)) as YvSwiGLUExpert._init_weights (expert.py:458-462)
    bound = 1.0 / math.sqrt(in_f)
    w = torch.empty(out_f, in_f, device=device)
    w.uniform_(-bound, bound, generator=generator)
    return w


class YvDynamicMoELayer(nn.Module):
    SKIP_RESIDUAL_WEIGHT = 0.1

    def __init__(self, cfg: Any, device=None, dtype=None, num_shared_experts: int = 1,
                 use_fine_grained: bool = False, num_sub_experts: int = 1,
                 compute_mode: str = "default", weight_format: Optional[str] = None,
                 router: Optional[str] = None):
        super().__init__()
        if compute_mode != "default":
            raise NotImplementedError("compute_split experts (layer.py:646-676) are not supported")
        self.cfg = cfg
        self.top_k = getattr(cfg, "moe_top_k", 8)
        self.num_experts = getattr(cfg, "moe_num_experts", 128)
        self.hidden_size = cfg.hidden_size
        self.intermediate_size = getattr(cfg, "intermediate_size", cfg.hidden_size * 4)
        self.num_shared_experts = num_shared_experts
        self.use_fine_grained = use_fine_grained
        self.num_sub_experts = num_sub_experts if use_fine_grained else 1
        self.compute_mode = compute_mode
        self.use_fused_moe = True
        self.dtype = dtype if dtype is not None else torch.float32
        if weight_format is None:
            weight_format = getattr(cfg, "moe_weight_format", None)
        if weight_format is None:
            weight_format = "bf16" if self.dtype == torch.bfloat16 else "f32"
        self.weight_format = FORMAT_BY_NAME[weight_format]
        H = self.hidden_size
        if router is None:
            router = getattr(cfg, "moe_router", "moegate")
        if router == "moegate":
            self.router = YvMoEGate(
                H, self.num_experts, top_k=self.top_k, device=device, dtype=dtype,
                load_balance_alpha=getattr(cfg, "moe_load_balance_alpha", 0.01),
                noise_std=getattr(cfg, "moe_noise_std", 0.1),
                enable_cognitive_density=getattr(cfg, "enable_cognitive_density", False), cfg=cfg)
        elif router == "stable":
            self.router = YvStableMoEGate(
                H, self.num_experts, top_k=self.top_k, device=device, dtype=dtype,
                capacity_factor=getattr(cfg, "moe_capacity_factor", 1.0),
                min_capacity=getattr(cfg, "moe_min_capacity", 4),
                prediction_horizon=getattr(cfg, "moe_prediction_horizon", 10),
                fixed_shape_mode=getattr(cfg, "moe_fixed_shape_mode", H <= 768),
                enable_dynamic_capacity=getattr(cfg, "enable_dynamic_capacity", True),
                enable_cognitive_density=getattr(cfg, "enable_cognitive_density", False))
        else:
            raise ValueError(f"router={router!r}: 'moegate' or 'stable'")
        self._router_kind = router
        self._router_mode = "token_gate"
        self._workspace: Optional[torch.Tensor] = None
        S = num_shared_experts
        self.experts_packed = self._random_experts(device)
        if S > 0:
            self.shared_expert_weight = nn.Parameter(
                torch.ones(S, device=device, dtype=dtype) / S)
        else:
            self.shared_expert_weight = None
        self._skip_buffer: Optional[torch.Tensor] = None
        self._step = 0
        self._mix_cache = None

    # ------------------------------------------------------------ weights
    def _random_experts(self, device) -> PackedExperts:
        H, Fd = self.hidden_size, self.intermediate_size
        pk = ExpertPacker(self.weight_format, self.num_experts, self.num_shared_experts, H, Fd,
                          device if device is not None else "cpu")
        for i in range(self.num_experts + self.num_shared_experts):
            pk.set(i, _kaiming_uniform(Fd, H, device=device), _kaiming_uniform(Fd, H, device=device),
                   _kaiming_uniform(H, Fd, device=device))
        return pk.packed

    def set_experts(self, packed: PackedExperts) -> None:
        if (packed.num_routed, packed.num_shared, packed.hidden, packed.ffn) != (
                self.num_experts, self.num_shared_experts, self.hidden_size, self.intermediate_size):
            raise ValueError("packed experts do not match the layer shape")
        self.experts_packed = packed
        self.weight_format = packed.format

    def _apply(self, fn, recurse=True):
        # packed experts follow the module's device; their dtypes are part of the format
        super()._apply(fn, recurse)
        p = self.experts_packed
        target = fn(torch.empty(0, device=p.w_gate.device)).device
        if target != p.w_gate.device:
            self.experts_packed = p.to(target)
        return self

    def load_reference_state_dict(self, sd: dict, strict: bool = False) -> None:
        """Load reference keys (layer.py:665-705, gate.py:920-1024) and pack the experts."""
        dev = self.router.gate.weight.device
        E, S = self.num_experts, self.num_shared_experts
        pk = ExpertPacker(self.weight_format, E, S, self.hidden_size, self.intermediate_size, dev)
        for i in range(E + S):
            pre = f"experts.{i}." if i < E else f"shared_experts.{i - E}.expert."
            ws = [sd[pre + f"{n}_proj.weight"] for n in ("gate", "up", "down")]
            pk.set(i, *[w.float() for w in ws])
        self.experts_packed = pk.packed
        if S > 0 and "shared_expert_weight" in sd:
            with torch.no_grad():
                self.shared_expert_weight.copy_(sd["shared_expert_weight"])
        router_sd = {k[len("router."):]: v for k, v in sd.items() if k.startswith("router.")}
        if router_sd:
            self.router.load_state_dict(router_sd, strict=strict)

    def load_packed(self, packed) -> None:
        """Load a packed layer: a file written by ``pisceslx_amd.checkpoint.convert`` (read onto
        the layer's device) or a ``checkpoint.PackedLayer``."""
        from .checkpoint import PackedLayer, load_packed
        dev = self.router.gate.weight.device
        pl = packed if isinstance(packed, PackedLayer) else load_packed(packed, device=dev)
        self.set_experts(pl.experts.to(dev))
        if self.shared_expert_weight is not None and pl.shared_expert_weight is not None:
            with torch.no_grad():
                self.shared_expert_weight.copy_(pl.shared_expert_weight)
        if pl.router:
            self.router.load_state_dict(pl.router, strict=False)

    def load_reference_checkpoint(self, path: str, prefix: str) -> None:
        """Load this layer's keys from a whole reference checkpoint (``.pt`` / ``.bin`` /
        ``.safetensors``, full-precision or reference-quantized experts), packing on the
        layer's device in its weight format."""
        from .checkpoint import StateSource, convert_layer, PackedLayer
        dev = self.router.gate.weight.device
        experts, router, sw = convert_layer(StateSource(path), prefix, FORMAT_NAMES[self.weight_format],
                                            device=dev)
        self.load_packed(PackedLayer(experts, router, sw, {}))

    # ------------------------------------------------------------ forward
    def _mix(self) -> Optional[torch.Tensor]:
        if self.shared_expert_weight is None:
            return None
        p = self.shared_expert_weight
        key = (p.data_ptr(), p._version)
        if self._mix_cache is None or self._mix_cache[0] != key:
            # softmax(shared_expert_weight) (layer.py:859) in the parameter's dtype, then fp32
            self._mix_cache = (key, F.softmax(p.detach(), dim=0).float().contiguous())
        return self._mix_cache[1]

    def _apply_skip_residual_buffer(self, shape) -> Optional[torch.Tensor]:
        buf = self._skip_buffer
        if buf is not None and tuple(buf.shape) == tuple(shape):
            return buf
        return None

    def forward(self, x: torch.Tensor, subconscious_hints: Optional[torch.Tensor] = None,
                modal_id: Optional[torch.Tensor] = None):
        if self.training:
            raise NotImplementedError("the MI355X Yv MoE layer is an inference forward; call .eval()")
        B, Sq, H = x.shape
        x2d = x.reshape(-1, H)
        if not x2d.is_contiguous():
            x2d = x2d.contiguous()
        act = yvf._act(x2d.dtype)
        has_shared = self.num_shared_experts > 0
        skip = None
        if has_shared:
            buf = self._apply_skip_residual_buffer((B, Sq, H))
            skip = None if buf is None else buf.reshape(-1, H)
        ws = self._workspace if self._workspace is not None and self._workspace.device == x.device else None
        if self._router_kind == "moegate":
            g = self.router
            st = g.gate_state(act, Sq)
            mid = None if modal_id is None else g._modal_ids(modal_id, B, Sq, x.device)
            cached = g.path_moe_begin(x2d.shape[0])
            out, shared_out, routing, logits, loss, ws = yvf.moe_forward_moegate(
                x2d, st, min(self.top_k, self.num_experts), self.experts_packed, self._mix(), skip,
                modal_id=mid, route_logits=None if cached is None else cached[0], workspace=ws)
            g.path_moe_end(None if cached is not None else (logits, routing))
            g.last_routing, g.last_logits, g._last_loss_f32 = routing, logits, loss
            loss = loss.reshape(()).to(x.dtype)
        else:
            st = self.router.router_state(act)
            if ws is None or ws.numel() < yvf.workspace_bytes(x2d.shape[0], act, st, self.experts_packed):
                ws = None
            out, shared_out, routing = yvf.moe_forward(x2d, st, self.experts_packed, self._mix(), skip,
                                                       workspace=ws)
            loss = torch.tensor(0.0, device=x.device, dtype=x.dtype)
        self._workspace = ws
        if has_shared:
            self._skip_buffer = shared_out.view(B, Sq, H)
        self.last_routing = routing
        self._step += 1
        return out.view(B, Sq, H), loss


class YvDeepSeekMoELayer(YvDynamicMoELayer):
    """YvDeepSeekMoELayer (layer.py:967): DeepSeek defaults read from cfg (layer.py:1040-1047).

    The diversity loss is training-only (layer.py:1385-1390); inference returns loss 0.
    ``expert_init_method`` only changes the random initialisation of experts, which a
    loaded state_dict replaces, so it is not reproduced.
    """

    def __init__(self, cfg: Any, device=None, dtype=None, weight_format: Optional[str] = None,
                 router: Optional[str] = None):
        super().__init__(cfg, device=device, dtype=dtype,
                         num_shared_experts=getattr(cfg, "moe_shared_experts", 1),
                         use_fine_grained=getattr(cfg, "moe_fine_grained", True),
                         num_sub_experts=getattr(cfg, "moe_num_sub_experts", 4),
                         compute_mode=getattr(cfg, "moe_compute_mode", "default"),
                         weight_format=weight_format, router=router)
        self.diversity_weight = getattr(cfg, "diversity_weight", 0.01)
