"""CPU oracle of the Yv MoE layer inference forward — TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may import this
module: as the checker of the GPU path, or (bench) as the timed reference CPU path. The
product package ``pisceslx_amd`` never imports it.

It restates the reference algorithm on the CPU with torch ops, following:

* ``YvStableMoEGate.forward`` model/moe/gate.py:1122-1247 — routing through the C oracle
  (route_oracle.c, which fixes the fp32 arithmetic so the GPU can match it bit for bit);
  the gate GEMM and ``_calculate_dynamic_capacity`` (gate.py:1096-1120) in float64,
  rounded to fp32;
* ``PiscesLxFusedMoEDispatch.forward`` opss/infer/fused_moe.py:54-123 — stable argsort,
  bincount offsets, a loop over active experts, then the weighted combine;
* ``YvSwiGLUExpert.forward`` model/moe/expert.py:475-489 — ``down(silu(gate(x)) * up(x))``
  with every ``F.linear`` correctly rounded to the layer dtype (exact float64 sum, one
  rounding; the reference's fp32 accumulation order is BLAS-dependent, so this is the
  order-free statement of the same rounding points), on weights dequantized inside the
  expert loop (bounded host memory);
* ``_compute_shared_expert_output`` model/moe/layer.py:812-865 — fused gate/up
  projection, ``softmax(shared_expert_weight)`` mixture;
* ``forward`` model/moe/layer.py:867-963 / :1283-1396 and ``_apply_skip_residual``
  :741-753 — ``routed + shared + 0.1 * skip``.

Where the reference leaves the dtype of the combine undefined (fp32 routing weights meet
bf16 expert outputs in ``index_add_``, fused_moe.py:117-119, which torch rejects), the
oracle accumulates the combine in fp32 and rounds once, as the GPU path does.

Parity status: routing (indices, weights, counts, offsets, perm, pos) is pinned by
tests/test_oracle_routing.py; the expert math and combine by closed-form float64 checks in
tests/test_oracle_layer.py.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch
import torch.nn.functional as F

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "libyvmoe_oracle.so")
_LIB = None


def build() -> str:
    """Compile the C oracle (gcc, no FMA contraction) into oracle/_build/."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _SO


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(_SO):
            build()
        l = ctypes.CDLL(_SO)
        fp, ip = ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_int32)
        l.yvo_expf.restype = ctypes.c_float
        l.yvo_expf.argtypes = [ctypes.c_float]
        l.yvo_expf_array.argtypes = [fp, fp, ctypes.c_int64]
        l.yvo_softmax_rows.argtypes = [fp, fp, ctypes.c_int, ctypes.c_int, fp]
        l.yvo_capacity.restype = ctypes.c_int
        l.yvo_capacity.argtypes = [ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        l.yvo_route.restype = ctypes.c_int
        l.yvo_route.argtypes = [fp, fp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                fp, fp, fp, ip, ctypes.POINTER(ctypes.c_uint8), ip, ip, ip, ip]
        _LIB = l
    return _LIB


def _fp(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _ip(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))


def expf(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().yvo_expf_array(_fp(x), _fp(y), x.size)
    return y


def softmax_rows(z: np.ndarray, bias: Optional[np.ndarray] = None) -> np.ndarray:
    z = np.ascontiguousarray(z, dtype=np.float32)
    N, E = z.shape
    p = np.empty_like(z)
    b = None if bias is None else _fp(np.ascontiguousarray(bias, dtype=np.float32))
    lib().yvo_softmax_rows(_fp(z), b, N, E, _fp(p))
    return p


def capacity(avg: float, n_tokens: int, num_experts: int, min_capacity: int) -> int:
    return int(lib().yvo_capacity(ctypes.c_float(avg), n_tokens, num_experts, min_capacity))


@dataclass
class OracleRouting:
    topp: np.ndarray      # [N,k] p of chosen experts
    w0: np.ndarray        # [N,k] weights before the capacity trim
    weights: np.ndarray   # [N,k] final weights
    indices: np.ndarray   # [N,k] int32
    allowed: np.ndarray   # [N,k] uint8
    counts: np.ndarray    # [E]
    offsets: np.ndarray   # [E+1]
    perm: np.ndarray      # [N*k]
    pos: np.ndarray       # [N*k]
    capacity: int


def route(logits: np.ndarray, k: int, cap: int, bias: Optional[np.ndarray] = None) -> OracleRouting:
    """Routing of fp32 logits [N, E]; cap < 0 = no capacity trim (fixed_shape_mode)."""
    z = np.ascontiguousarray(logits, dtype=np.float32)
    N, E = z.shape
    f32 = lambda *s: np.empty(s, dtype=np.float32)
    i32 = lambda *s: np.empty(s, dtype=np.int32)
    topp, w0, w = f32(N, k), f32(N, k), f32(N, k)
    idx = i32(N, k)
    allowed = np.empty((N, k), dtype=np.uint8)
    counts, offsets = i32(E), i32(E + 1)
    perm, pos = i32(N * k), i32(N * k)
    b = None if bias is None else _fp(np.ascontiguousarray(bias, dtype=np.float32))
    rc = lib().yvo_route(_fp(z), b, N, E, k, cap, _fp(topp), _fp(w0), _fp(w), _ip(idx),
                         allowed.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), _ip(counts),
                         _ip(offsets), _ip(perm), _ip(pos))
    if rc != 0:
        raise ValueError(f"yvo_route rejected N={N} E={E} k={k}")
    return OracleRouting(topp, w0, w, idx, allowed, counts, offsets, perm, pos, cap)


# ------------------------------------------------------------------ layer parameters
@dataclass
class LayerParams:
    """Dense (dequantized) view of one Yv MoE layer for the oracle.

    expert(i) returns (Wg [F,H], Wu [F,H], Wd [H,F]) of routed expert i (i < E) or shared
    expert i - E, as fp32 tensors dequantized on demand.
    """

    hidden: int
    ffn: int
    num_experts: int
    num_shared: int
    top_k: int
    gate_weight: torch.Tensor          # [E, H] (gate dtype)
    pred: Optional[Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]]  # W1, b1, W2, b2
    bias: Optional[torch.Tensor]       # [E] fp32 added to logits (fixed mode) or None
    fixed_shape_mode: bool
    dynamic_capacity: bool
    capacity_factor: float
    min_capacity: int
    mix_param: Optional[torch.Tensor]  # shared_expert_weight [S]
    expert_fn: object                  # callable i -> (Wg, Wu, Wd) fp32

    def expert(self, i: int):
        return self.expert_fn(i)


def params_from_workload(w) -> LayerParams:
    """Oracle view of a pisceslx_amd.workloads.Workload (weights copied to the host and
    dequantized per expert on demand)."""
    cpu = w.experts.to("cpu")
    spec = w.spec
    pred = None if w.pred is None else tuple(t.detach().cpu() for t in w.pred)
    return LayerParams(
        hidden=spec.hidden, ffn=spec.ffn, num_experts=spec.num_experts, num_shared=spec.num_shared,
        top_k=spec.top_k, gate_weight=w.gate_weight.cpu(), pred=pred,
        bias=None if w.expert_bias is None else w.expert_bias.cpu(),
        fixed_shape_mode=spec.fixed_shape_mode, dynamic_capacity=not spec.fixed_shape_mode,
        capacity_factor=1.0, min_capacity=4,
        mix_param=None if w.shared_expert_weight is None else w.shared_expert_weight.cpu(),
        expert_fn=lambda i: cpu.dequantize(i, torch.float32))


def router_logits(x2d: torch.Tensor, gate_weight: torch.Tensor) -> np.ndarray:
    """gate(x_flat) (gate.py:1179) in float64, rounded to fp32 logits."""
    return (x2d.double() @ gate_weight.double().t()).float().numpy()


def complexity_scores(x2d: torch.Tensor, pred) -> torch.Tensor:
    """complexity_predictor(x) (gate.py:930-936, :1112-1116) in float64 -> fp32 [N]."""
    W1, b1, W2, b2 = pred
    h = torch.relu(x2d.double() @ W1.double().t() + b1.double())
    return torch.sigmoid(h @ W2.double().reshape(-1, 1) + b2.double()).reshape(-1).float()


def layer_capacity(params: LayerParams, x2d: torch.Tensor) -> int:
    """tokens_per_expert of gate.py:1172-1176."""
    N = x2d.shape[0]
    E = params.num_experts
    if params.dynamic_capacity:
        avg = float(complexity_scores(x2d, params.pred).mean()) if N > 0 else float("nan")
        if N == 0:
            return params.min_capacity
        return capacity(avg, N, E, params.min_capacity)
    c = int(N * params.capacity_factor / E)
    return max(c, params.min_capacity)


def linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """F.linear(x, w) of the layer dtype, correctly rounded: the exact (float64) sum rounded
    once to x's dtype. The reference's F.linear accumulates in fp32 in a BLAS-dependent
    order; the correctly rounded product is the order-free statement of the same rounding
    point, so any fp32 implementation differs from it only by its own accumulation error."""
    return (x.double() @ w.double().t()).to(x.dtype)


def swiglu(xs: torch.Tensor, wg: torch.Tensor, wu: torch.Tensor, wd: torch.Tensor, lin=linear) -> torch.Tensor:
    """YvSwiGLUExpert.forward (expert.py:484-489) in the dtype of its inputs."""
    return lin(F.silu(lin(xs, wg)) * lin(xs, wu), wd)


@dataclass
class OracleDispatch:
    out: torch.Tensor        # [N, H] in x's dtype
    counts: np.ndarray       # [E]
    offsets: np.ndarray      # [E+1]
    perm: np.ndarray         # [V] flat slots of the valid slots in expert-sorted order
    Y: torch.Tensor          # [V, H] fp32 expert outputs (values of x's dtype) in that order
    invalid: int             # slots whose index lies outside [0, E)


def dispatch_forward(x2d: torch.Tensor, weights, indices, num_experts: int, expert_fn,
                     tokens: Optional[np.ndarray] = None, lin=None) -> OracleDispatch:
    """``PiscesLxFusedMoEDispatch.forward`` (opss/infer/fused_moe.py:54-123) given the
    routing: ``token_ids = arange(N).repeat_interleave(k)`` (:83-84), a stable argsort of the
    flat indices (:87), ``bincount`` / ``cumsum`` offsets (:93-95), the gathered rows of each
    active expert through ``YvSwiGLUExpert.forward`` (:103-111) — ``expert_fn(e)`` returns its
    (Wg, Wu, Wd) as fp32 — and the weighted combine (:117-119), summed per token in fp32 in
    slot order and rounded once to x's dtype (the build's statement of the index_add_, whose
    dtype and order the reference leaves to torch). Slots with an index outside [0, E) are
    counted in ``invalid`` and add nothing (the reference raises on them). ``tokens``
    restricts the expert math to a subset of tokens (other rows stay zero)."""
    lin = linear if lin is None else lin
    dtype = x2d.dtype
    N, H = x2d.shape
    idx = np.asarray(indices, dtype=np.int64).reshape(N, -1)
    k = idx.shape[1]
    w = torch.as_tensor(np.asarray(weights, dtype=np.float32)).reshape(N, k)
    flat = idx.reshape(-1)
    ok = (flat >= 0) & (flat < num_experts)
    valid_slots = np.nonzero(ok)[0]
    order = np.argsort(flat[valid_slots], kind="stable")
    perm = valid_slots[order].astype(np.int64)
    counts = np.bincount(flat[valid_slots], minlength=num_experts).astype(np.int64)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    keep = np.ones(N, dtype=bool)
    if tokens is not None:
        keep[:] = False
        keep[np.asarray(tokens)] = True
    token_of = perm // k
    Y = torch.zeros(len(perm), H, dtype=torch.float32)
    for e in range(num_experts):
        a, b = int(offsets[e]), int(offsets[e + 1])
        sel = np.arange(a, b)[keep[token_of[a:b]]]
        if len(sel) == 0:
            continue
        rows = torch.from_numpy(token_of[sel])
        wg, wu, wd = expert_fn(e)
        Y[torch.from_numpy(sel)] = swiglu(x2d[rows], wg.to(dtype), wu.to(dtype), wd.to(dtype), lin).float()
    pos = np.full(N * k, -1, dtype=np.int64)
    pos[perm] = np.arange(len(perm))
    acc = torch.zeros(N, H, dtype=torch.float32)
    pos_t = torch.from_numpy(pos.reshape(N, k))
    for j in range(k):
        live = pos_t[:, j] >= 0
        rows = torch.nonzero(live).reshape(-1)
        if len(rows):
            acc[rows] = acc[rows] + w[rows, j:j + 1] * Y[pos_t[rows, j]]
    return OracleDispatch(acc.to(dtype), counts, offsets, perm, Y, int((~ok).sum()))


def layer_forward(x2d: torch.Tensor, params: LayerParams, logits: Optional[np.ndarray] = None,
                  cap: Optional[int] = None, skip: Optional[torch.Tensor] = None,
                  routing: Optional[OracleRouting] = None,
                  tokens: Optional[np.ndarray] = None,
                  reference_linear: bool = False) -> Dict[str, object]:
    """Reference forward of one packed batch x2d [N, H] (CPU, layer dtype = x2d.dtype).

    logits / cap / routing may be supplied to check the GPU path "given identical fp32 gate
    logits". ``tokens`` restricts the expert math to a subset of tokens (rows of other
    tokens are left zero): given the routing, tokens are independent. Returns out [N,H],
    shared [N,H] (or None) and the routing. ``reference_linear`` runs the GEMMs as the
    reference does on the CPU (``F.linear`` in the layer dtype, torch's own accumulation
    order) instead of correctly rounded: the timed CPU baseline uses it, the checks do not.
    """
    lin = (lambda a, b: F.linear(a, b)) if reference_linear else linear
    dtype = x2d.dtype
    N, H = x2d.shape
    E, S, k = params.num_experts, params.num_shared, params.top_k
    if routing is None:
        if logits is None:
            logits = router_logits(x2d, params.gate_weight)
        if params.fixed_shape_mode:
            c = -1
        else:
            c = layer_capacity(params, x2d) if cap is None else cap
        bias = None if params.bias is None else params.bias.float().numpy()
        routing = route(logits, k, c, bias)
    # dispatch (fused_moe.py:83-119): stable sort by expert, loop over active experts
    token_of = routing.perm // k
    keep = np.ones(N, dtype=bool)
    if tokens is not None:
        keep[:] = False
        keep[np.asarray(tokens)] = True
    Y = torch.zeros(N * k, H, dtype=torch.float32)   # expert outputs in expert-sorted order
    for e in range(E):
        a, b = int(routing.offsets[e]), int(routing.offsets[e + 1])
        sel = np.arange(a, b)[keep[token_of[a:b]]]
        if len(sel) == 0:
            continue
        rows = torch.from_numpy(token_of[sel].astype(np.int64))
        wg, wu, wd = params.expert(e)
        ye = swiglu(x2d[rows], wg.to(dtype), wu.to(dtype), wd.to(dtype), lin)
        Y[torch.from_numpy(sel)] = ye.float()
    # weighted combine (fused_moe.py:117-119): per token, slots j = 0..k-1 in order,
    # multiply then add in fp32 (the reference's GPU index_add_ is atomic and unordered)
    acc = torch.zeros(N, H, dtype=torch.float32)
    pos = torch.from_numpy(routing.pos.reshape(N, k).astype(np.int64))
    wts = torch.from_numpy(routing.weights.reshape(N, k))
    for j in range(k):
        acc = acc + wts[:, j:j + 1] * Y[pos[:, j]]
    # the routed sum accumulates in fp32 and is rounded once to the layer dtype (the
    # reference's index_add_ of fp32 weights into a bf16 output is undefined); the shared
    # mixture and the residual adds are tensor ops of the layer dtype (layer.py:859-863,
    # :942-945, :750-752), rounded after every step
    out = acc.to(dtype)
    shared = None
    if S > 0:
        mix = F.softmax(params.mix_param.detach(), dim=0)
        shared = torch.zeros(N, H, dtype=dtype)
        rows = torch.from_numpy(np.nonzero(keep)[0])
        for s in range(S):
            wg, wu, wd = params.expert(E + s)
            wf = torch.cat([wg, wu], dim=0).to(dtype)  # layer.py:844 fused gate/up
            g, u = lin(x2d[rows], wf).chunk(2, dim=-1)
            so = lin(F.silu(g) * u, wd.to(dtype))
            shared[rows] = shared[rows] + mix[s].to(dtype) * so
        out = out + shared
        if skip is not None and tuple(skip.shape) == (N, H):
            out = out + 0.1 * skip.to(dtype)
    return {"out": out, "shared": shared,
            "routing": routing, "logits": logits}
