"""Functional entry points over libyvmoe: torch allocates, the HIP library computes.

Every function runs on the tensors' CUDA (HIP) device and on torch's current stream; none
of them has a CPU or PyTorch fallback — a call on CPU tensors raises.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from .quant import PackedExperts


def _act(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return _lib.ACT_BF16
    if dtype == torch.float32:
        return _lib.ACT_F32
    raise ValueError(f"activation dtype {dtype} is not supported (bfloat16 or float32)")


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _stream(device: torch.device):
    return torch.cuda.current_stream(device).cuda_stream


def _require_cuda(*ts: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("libyvmoe computes on the GPU only: got a CPU tensor")
        if not t.is_contiguous():
            raise ValueError("libyvmoe needs contiguous tensors")
        dev = t.device
    return dev


def router_ld(num_experts: int, act: int) -> int:
    ep = (num_experts + 15) // 16 * 16
    return ep + (3 if act == _lib.ACT_BF16 else 1) * _lib.PREDICTOR_DIM


@dataclass
class RouterState:
    """Device tensors of one YvStableMoEGate, packed for the router GEMM."""

    num_experts: int
    hidden: int
    top_k: int
    fixed_shape_mode: bool
    dynamic_capacity: bool
    min_capacity: int
    capacity_factor: float
    w_router: torch.Tensor
    b1: Optional[torch.Tensor]
    w2: Optional[torch.Tensor]
    b2: Optional[torch.Tensor]
    bias: Optional[torch.Tensor]

    def struct(self) -> _lib.Router:
        return _lib.Router(self.num_experts, self.hidden, self.top_k, int(self.fixed_shape_mode),
                           int(self.dynamic_capacity), self.min_capacity, float(self.capacity_factor),
                           _ptr(self.w_router), _ptr(self.b1), _ptr(self.w2), _ptr(self.b2),
                           _ptr(self.bias))


@dataclass
class Routing:
    weights: torch.Tensor   # [N, k] fp32
    indices: torch.Tensor   # [N, k] int64
    counts: torch.Tensor    # [E] int32
    offsets: torch.Tensor   # [E+1] int32
    perm: torch.Tensor      # [N*k] int32
    pos: torch.Tensor       # [N*k] int32
    capacity: torch.Tensor  # [1] int32

    @staticmethod
    def empty(N: int, E: int, k: int, device) -> "Routing":
        i32 = dict(dtype=torch.int32, device=device)
        return Routing(torch.empty(N, k, dtype=torch.float32, device=device),
                       torch.empty(N, k, dtype=torch.int64, device=device),
                       torch.empty(E, **i32), torch.empty(E + 1, **i32),
                       torch.empty(N * k, **i32), torch.empty(N * k, **i32),
                       torch.empty(1, **i32))

    def struct(self) -> _lib.Routing:
        return _lib.Routing(self.weights.data_ptr(), self.indices.data_ptr(), self.counts.data_ptr(),
                            self.offsets.data_ptr(), self.perm.data_ptr(), self.pos.data_ptr(),
                            self.capacity.data_ptr())


def workspace_bytes(n_tokens: int, act: int, router: RouterState,
                    experts: Optional[PackedExperts] = None) -> int:
    r = router.struct()
    e = experts.struct() if experts is not None else None
    return int(_lib.lib().yvmoe_workspace_bytes(n_tokens, act, ctypes.byref(r),
                                                ctypes.byref(e) if e is not None else None))


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)


def router_logits(x2d: torch.Tensor, router: RouterState) -> torch.Tensor:
    """[N, ld] fp32: gate logits in columns [0, E), predictor first-layer terms after Ep."""
    dev = _require_cuda(x2d, router.w_router)
    act = _act(x2d.dtype)
    N = x2d.shape[0]
    ld = router_ld(router.num_experts, act)
    out = torch.empty(N, ld, dtype=torch.float32, device=dev)
    r = router.struct()
    ws = _workspace(int(_lib.lib().yvmoe_router_workspace_bytes(N, act, ctypes.byref(r))), dev)
    _lib.check(_lib.lib().yvmoe_router_logits(x2d.data_ptr(), act, N, ctypes.byref(r),
                                               out.data_ptr(), ld, ws.data_ptr(), ws.numel(),
                                               _stream(dev)),
               "yvmoe_router_logits")
    return out


def route(logits: torch.Tensor, router: RouterState, predictor: bool = True,
          capacity_override: int = -1) -> Routing:
    """Routing from fp32 logits [N, ld] (first E columns are the gate logits).

    ``predictor`` says the predictor columns follow at column Ep (as router_logits returns);
    pass False for plain [N, E] logits together with a capacity override or a fixed-mode gate.
    """
    dev = _require_cuda(logits)
    if logits.dtype != torch.float32:
        raise ValueError("routing needs fp32 logits")
    N, ld = logits.shape
    E, k = router.num_experts, router.top_k
    out = Routing.empty(N, E, k, dev)
    ws = _workspace(workspace_bytes(N, _lib.ACT_F32, router), dev)
    r = router.struct()
    o = out.struct()
    Ep = (E + 15) // 16 * 16
    pred_ptr = logits.data_ptr() + Ep * 4 if (predictor and N > 0) else None
    _lib.check(_lib.lib().yvmoe_route(logits.data_ptr() if N > 0 else None, ld, pred_ptr, N,
                                       ctypes.byref(r), capacity_override, ctypes.byref(o),
                                       ws.data_ptr(), ws.numel(), _stream(dev)), "yvmoe_route")
    return out


def expert_ffn(x2d: torch.Tensor, experts: PackedExperts, routing: Routing, top_k: int,
               workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y [N*k + S*N, H]: expert outputs in expert-sorted order, then the shared experts.

    Reads the routing's offsets and permutation only; ``workspace`` is scratch (allocated
    here when None or too small)."""
    dev = _require_cuda(x2d, *experts.tensors())
    act = _act(x2d.dtype)
    N = x2d.shape[0]
    R = N * top_k + experts.num_shared * N
    y = torch.empty(R, experts.hidden, dtype=x2d.dtype, device=dev)
    e = experts.struct()
    o = routing.struct()
    r = _lib.Router(experts.num_routed, experts.hidden, top_k, 0, 0, 0, 1.0, None, None, None,
                    None, None)
    need = int(_lib.lib().yvmoe_workspace_bytes(N, act, ctypes.byref(r), ctypes.byref(e)))
    if workspace is None or workspace.numel() < need:
        workspace = _workspace(need, dev)
    _lib.check(_lib.lib().yvmoe_expert_ffn(x2d.data_ptr(), act, N, top_k, ctypes.byref(e),
                                            ctypes.byref(o), y.data_ptr(), workspace.data_ptr(),
                                            workspace.numel(), _stream(dev)), "yvmoe_expert_ffn")
    return y


def dispatch_workspace_bytes(n_tokens: int, act: int, slots: int, experts: PackedExperts) -> int:
    e = experts.struct()
    return int(_lib.lib().yvmoe_dispatch_workspace_bytes(n_tokens, act, slots, ctypes.byref(e)))


def dispatch(x2d: torch.Tensor, routing_weights: torch.Tensor, expert_indices: torch.Tensor,
             experts: PackedExperts, want_expert_outputs: bool = False,
             workspace: Optional[torch.Tensor] = None):
    """Dispatch of an external routing (yvmoe_dispatch): grouped SwiGLU of the routed experts
    over every (token, slot) of ``expert_indices`` [N, k] int64 with ``routing_weights``
    [N, k] (fp32 or bf16), combined per token. Nothing synchronizes with the host.

    Returns (out [N, H], counts [E] int32, offsets [E+1] int32, invalid [1] int32 = number of
    slots whose index lies outside [0, E), expert outputs [N*k, H] in expert-sorted order or
    None).
    """
    dev = _require_cuda(x2d, routing_weights, expert_indices, *experts.tensors())
    act = _act(x2d.dtype)
    N, H = x2d.shape
    if H != experts.hidden:
        raise ValueError(f"hidden size {H} does not match the experts ({experts.hidden})")
    if expert_indices.dtype != torch.int64 or expert_indices.dim() != 2 or expert_indices.shape[0] != N:
        raise ValueError("expert_indices must be int64 [N, k]")
    k = expert_indices.shape[1]
    if tuple(routing_weights.shape) != (N, k):
        raise ValueError(f"routing_weights must be [N, k] = [{N}, {k}]")
    wdt = _act(routing_weights.dtype)
    E = experts.num_routed
    out = torch.empty_like(x2d)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    invalid = torch.empty(1, dtype=torch.int32, device=dev)
    y = torch.empty(N * k, H, dtype=x2d.dtype, device=dev) if want_expert_outputs else None
    need = dispatch_workspace_bytes(N, act, k, experts)
    if need == 0:
        raise ValueError(f"yvmoe_dispatch_workspace_bytes rejected k={k}")
    if workspace is None or workspace.numel() < need:
        workspace = _workspace(need, dev)
    e = experts.struct()
    _lib.check(_lib.lib().yvmoe_dispatch(
        x2d.data_ptr() if N > 0 else None, act, N,
        routing_weights.data_ptr() if N > 0 else None, wdt,
        expert_indices.data_ptr() if N > 0 else None, k, ctypes.byref(e),
        out.data_ptr() if N > 0 else None, _ptr(y) if N > 0 else None, counts.data_ptr(),
        offsets.data_ptr(), invalid.data_ptr(), workspace.data_ptr(), workspace.numel(),
        _stream(dev)), "yvmoe_dispatch")
    return out, counts, offsets, invalid, y


def moe_forward(x2d: torch.Tensor, router: RouterState, experts: PackedExperts,
                mix: Optional[torch.Tensor], skip: Optional[torch.Tensor],
                workspace: Optional[torch.Tensor] = None):
    """Whole layer. Returns (out [N,H], shared_out [N,H] or None, Routing)."""
    dev = _require_cuda(x2d, router.w_router, mix, skip, *experts.tensors())
    act = _act(x2d.dtype)
    N, H = x2d.shape
    if H != experts.hidden or H != router.hidden:
        raise ValueError(f"hidden size {H} does not match the layer ({experts.hidden})")
    E, k, S = router.num_experts, router.top_k, experts.num_shared
    routing = Routing.empty(N, E, k, dev)
    out = torch.empty_like(x2d)
    shared_out = torch.empty_like(x2d) if S > 0 else None
    need = workspace_bytes(N, act, router, experts)
    if workspace is None or workspace.numel() < need:
        workspace = _workspace(need, dev)
    if skip is not None and (skip.shape != x2d.shape or skip.dtype != x2d.dtype):
        raise ValueError("skip buffer must match x")
    if mix is not None and (mix.dtype != torch.float32 or mix.numel() != S):
        raise ValueError("mix must be fp32 [S]")
    r = router.struct()
    e = experts.struct()
    o = routing.struct()
    _lib.check(_lib.lib().yvmoe_forward(x2d.data_ptr(), act, N, ctypes.byref(r), ctypes.byref(e),
                                         _ptr(mix), _ptr(skip), out.data_ptr(), _ptr(shared_out),
                                         ctypes.byref(o), workspace.data_ptr(), workspace.numel(),
                                         _stream(dev)), "yvmoe_forward")
    return out, shared_out, routing


def moe_forward_static(x2d: torch.Tensor, router: RouterState, experts: PackedExperts,
                       mix: Optional[torch.Tensor], skip: Optional[torch.Tensor],
                       out: Optional[torch.Tensor] = None,
                       shared_out: Optional[torch.Tensor] = None,
                       routing: Optional[Routing] = None):
    """Whole layer on the library's own static scratch (yvmoe_forward_static): the library
    call allocates no device memory. Pass ``out``, ``shared_out`` and ``routing`` to make the
    whole call allocation-free (otherwise they are allocated here, before the library call).
    Calls that overlap on one GPU share its scratch and race. Returns (out, shared_out or
    None, Routing)."""
    dev = _require_cuda(x2d, router.w_router, mix, skip, out, shared_out, *experts.tensors())
    act = _act(x2d.dtype)
    N, H = x2d.shape
    if H != experts.hidden or H != router.hidden:
        raise ValueError(f"hidden size {H} does not match the layer ({experts.hidden})")
    E, k, S = router.num_experts, router.top_k, experts.num_shared
    if skip is not None and (skip.shape != x2d.shape or skip.dtype != x2d.dtype):
        raise ValueError("skip buffer must match x")
    if mix is not None and (mix.dtype != torch.float32 or mix.numel() != S):
        raise ValueError("mix must be fp32 [S]")
    if routing is None:
        routing = Routing.empty(N, E, k, dev)
    if out is None:
        out = torch.empty_like(x2d)
    if shared_out is None and S > 0:
        shared_out = torch.empty_like(x2d)
    for t in (out, shared_out):
        if t is not None and (t.shape != x2d.shape or t.dtype != x2d.dtype):
            raise ValueError("out and shared_out must match x")
    r = router.struct()
    e = experts.struct()
    o = routing.struct()
    _lib.check(_lib.lib().yvmoe_forward_static(x2d.data_ptr(), act, N, ctypes.byref(r),
                                                ctypes.byref(e), _ptr(mix), _ptr(skip),
                                                out.data_ptr(), _ptr(shared_out) if S > 0 else None,
                                                ctypes.byref(o), _stream(dev)),
               "yvmoe_forward_static")
    return out, (shared_out if S > 0 else None), routing


@dataclass
class MoEGateState:
    """Device tensors and constants of one YvMoEGate, regrouped for yvmoe_moegate_logits."""

    num_experts: int
    hidden: int
    enc_dim: int
    dg_dim: int
    sparsity_k: int
    n_modalities: int
    heads: int                      # _lib.HEAD_* bits
    w_proj: torch.Tensor            # [(dg if HiCL) + Rh, H] activation dtype
    dg_bias: Optional[torch.Tensor]
    prototypes_t: Optional[torch.Tensor]
    eo_mat: Optional[torch.Tensor]  # [D, E] fp32
    modal_affinity: Optional[torch.Tensor]
    expert_bias: Optional[torch.Tensor]
    w_hicl: float
    w_got: float
    w_soft: float
    w_eo: float
    soft_temperature: float
    temperature: float
    soft_eps: float
    load_balance_alpha: float
    z_loss_alpha: float
    soft_budget: float
    capacity_loss: float

    def tensors(self):
        return [t for t in (self.w_proj, self.dg_bias, self.prototypes_t, self.eo_mat,
                            self.modal_affinity, self.expert_bias)
                if t is not None]

    def struct(self) -> _lib.MoEGate:
        return _lib.MoEGate(
            self.num_experts, self.hidden, self.enc_dim, self.dg_dim, self.sparsity_k,
            self.n_modalities, self.heads, 0, _ptr(self.w_proj), _ptr(self.dg_bias), _ptr(self.prototypes_t), _ptr(self.eo_mat),
            _ptr(self.modal_affinity), _ptr(self.expert_bias),
            self.w_hicl, self.w_got, self.w_soft, self.w_eo, self.soft_temperature,
            self.temperature, self.soft_eps, self.load_balance_alpha, self.z_loss_alpha,
            self.soft_budget, self.capacity_loss, 0.0)


def moegate_workspace_bytes(n_tokens: int, act: int, gate: MoEGateState) -> int:
    g = gate.struct()
    return int(_lib.lib().yvmoe_moegate_workspace_bytes(n_tokens, act, ctypes.byref(g)))


def moegate_logits(x2d: torch.Tensor, gate: MoEGateState, modal_id: Optional[torch.Tensor] = None,
                   workspace: Optional[torch.Tensor] = None):
    """YvMoEGate logits [N, E] fp32 (temperature-scaled) and the routing loss [1] fp32."""
    dev = _require_cuda(x2d, modal_id, *gate.tensors())
    act = _act(x2d.dtype)
    N, H = x2d.shape
    if H != gate.hidden:
        raise ValueError(f"hidden size {H} does not match the gate ({gate.hidden})")
    if modal_id is not None and (modal_id.dtype != torch.int32 or modal_id.numel() != N):
        raise ValueError("modal_id must be int32 [N]")
    E = gate.num_experts
    logits = torch.empty(N, E, dtype=torch.float32, device=dev)
    loss = torch.empty(1, dtype=torch.float32, device=dev)
    need = moegate_workspace_bytes(N, act, gate)
    if need == 0:
        raise ValueError("yvmoe_moegate_workspace_bytes rejected the gate state")
    if workspace is None or workspace.numel() < need:
        workspace = _workspace(need, dev)
    g = gate.struct()
    _lib.check(_lib.lib().yvmoe_moegate_logits(x2d.data_ptr() if N > 0 else None, act, N,
                                                ctypes.byref(g), _ptr(modal_id),
                                                logits.data_ptr() if N > 0 else None,
                                                loss.data_ptr(), workspace.data_ptr(),
                                                workspace.numel(), _stream(dev)),
               "yvmoe_moegate_logits")
    return logits, loss


def moegate_forward(x2d: torch.Tensor, gate: MoEGateState, top_k: int,
                    modal_id: Optional[torch.Tensor] = None,
                    workspace: Optional[torch.Tensor] = None):
    """YvMoEGate logits [N, E], loss [1] and the fixed-mode routing, in one library call.

    Returns (logits, loss, Routing, workspace); the routing can be passed on to expert_ffn.
    """
    dev = _require_cuda(x2d, modal_id, *gate.tensors())
    act = _act(x2d.dtype)
    N, H = x2d.shape
    if H != gate.hidden:
        raise ValueError(f"hidden size {H} does not match the gate ({gate.hidden})")
    if modal_id is not None and (modal_id.dtype != torch.int32 or modal_id.numel() != N):
        raise ValueError("modal_id must be int32 [N]")
    E = gate.num_experts
    g = gate.struct()
    need = int(_lib.lib().yvmoe_moegate_forward_workspace_bytes(N, act, top_k, ctypes.byref(g)))
    if need == 0:
        raise ValueError("yvmoe_moegate_forward_workspace_bytes rejected the gate state / top_k")
    if workspace is None or workspace.numel() < need:
        workspace = _workspace(need, dev)
    logits = torch.empty(N, E, dtype=torch.float32, device=dev)
    loss = torch.empty(1, dtype=torch.float32, device=dev)
    routing = Routing.empty(N, E, top_k, dev)
    o = routing.struct()
    _lib.check(_lib.lib().yvmoe_moegate_forward(x2d.data_ptr() if N > 0 else None, act, N,
                                                 ctypes.byref(g), _ptr(modal_id), top_k,
                                                 logits.data_ptr() if N > 0 else None,
                                                 loss.data_ptr(), ctypes.byref(o),
                                                 workspace.data_ptr(), workspace.numel(),
                                                 _stream(dev)), "yvmoe_moegate_forward")
    return logits, loss, routing, workspace


def moe_forward_moegate(x2d: torch.Tensor, gate: MoEGateState, top_k: int, experts: PackedExperts,
                        mix: Optional[torch.Tensor], skip: Optional[torch.Tensor],
                        modal_id: Optional[torch.Tensor] = None,
                        route_logits: Optional[torch.Tensor] = None,
                        workspace: Optional[torch.Tensor] = None):
    """Whole layer with a YvMoEGate router. Returns (out, shared_out or None, Routing, logits,
    loss, workspace); ``route_logits`` (fp32 [N, E]) routes on earlier logits instead."""
    dev = _require_cuda(x2d, mix, skip, modal_id, route_logits, *gate.tensors(), *experts.tensors())
    act = _act(x2d.dtype)
    N, H = x2d.shape
    if H != experts.hidden or H != gate.hidden:
        raise ValueError(f"hidden size {H} does not match the layer ({experts.hidden})")
    if skip is not None and (skip.shape != x2d.shape or skip.dtype != x2d.dtype):
        raise ValueError("skip buffer must match x")
    if mix is not None and (mix.dtype != torch.float32 or mix.numel() != experts.num_shared):
        raise ValueError("mix must be fp32 [S]")
    if modal_id is not None and (modal_id.dtype != torch.int32 or modal_id.numel() != N):
        raise ValueError("modal_id must be int32 [N]")
    E, S = gate.num_experts, experts.num_shared
    if route_logits is not None and (route_logits.dtype != torch.float32 or
                                     tuple(route_logits.shape) != (N, E)):
        raise ValueError("route_logits must be fp32 [N, E]")
    g = gate.struct()
    e = experts.struct()
    need = int(_lib.lib().yvmoe_forward_moegate_workspace_bytes(N, act, top_k, ctypes.byref(g),
                                                                ctypes.byref(e)))
    if need == 0:
        raise ValueError("yvmoe_forward_moegate_workspace_bytes rejected the gate / experts / top_k")
    if workspace is None or workspace.numel() < need:
        workspace = _workspace(need, dev)
    routing = Routing.empty(N, E, top_k, dev)
    out = torch.empty_like(x2d)
    shared_out = torch.empty_like(x2d) if S > 0 else None
    logits = torch.empty(N, E, dtype=torch.float32, device=dev)
    loss = torch.empty(1, dtype=torch.float32, device=dev)
    o = routing.struct()
    _lib.check(_lib.lib().yvmoe_forward_moegate(
        x2d.data_ptr() if N > 0 else None, act, N, ctypes.byref(g), _ptr(modal_id), top_k,
        _ptr(route_logits), ctypes.byref(e), _ptr(mix), _ptr(skip),
        out.data_ptr() if N > 0 else None, _ptr(shared_out) if N > 0 else None, ctypes.byref(o),
        logits.data_ptr() if N > 0 else None, loss.data_ptr(), workspace.data_ptr(),
        workspace.numel(), _stream(dev)), "yvmoe_forward_moegate")
    return out, shared_out, routing, logits, loss, workspace


def rms_norm(x: torch.Tensor, norms, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """RMSNorm over the last dimension, one or two norms in sequence in one pass.

    ``norms`` is a sequence of (weight, bias or None, eps); two entries apply the second norm to
    the first one's output rounded to x's dtype (YvHybridBlock's norm_fusion then norm_mlp,
    model/core/hybrid.py:1359, :1310). Each norm follows fused_rms_norm
    (opss/kernels/fused_rms_norm.py:42): fp32 sum of squares, (x / sqrt(Σx²/H + eps)) * weight
    rounded once, + bias rounded again (model/core/norms.py:998-999). ``out`` may be x.
    """
    norms = list(norms)
    if len(norms) not in (1, 2):
        raise ValueError("rms_norm takes one or two norms")
    H = x.shape[-1]
    ts = [x] + [t for w, b, _ in norms for t in (w, b)]
    dev = _require_cuda(*ts, out)
    act = _act(x.dtype)
    for w, b, _ in norms:
        for t in (w, b):
            if t is not None and (t.dtype != x.dtype or t.numel() != H):
                raise ValueError(f"norm weight/bias must be {x.dtype} [{H}]")
    if out is None:
        out = torch.empty_like(x)
    elif out.shape != x.shape or out.dtype != x.dtype:
        raise ValueError("out must match x")
    N = x.numel() // H if H else 0
    params = (_lib.RMSNormParams * len(norms))()
    for i, (w, b, eps) in enumerate(norms):
        params[i].weight = w.data_ptr()
        params[i].bias = _ptr(b)
        params[i].eps = float(eps)
    _lib.check(_lib.lib().yvmoe_rmsnorm(x.data_ptr() if N > 0 else None, act, N, H, params,
                                        len(norms), out.data_ptr() if N > 0 else None,
                                        _stream(dev)), "yvmoe_rmsnorm")
    return out
