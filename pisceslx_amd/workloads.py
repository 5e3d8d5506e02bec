"""Seeded synthetic workloads of the five benchmark configurations.

Each configuration is a Yv MoE layer shape, a weight format and a packed ragged batch:

  cfg1  H1024 E8   F2816 top-2 S1 fp32 (unquantized), 16 sequences, lengths U[1,256] (N=2052)
  cfg2  H4096 E64  F1408 top-6 S2 W8A16 int8, decode 64 x 1 token
  cfg3  same layer as cfg2, ragged prefill: 32 sequences, log-normal(6, 0.8) clipped
        [16, 2048], about 16K tokens
  cfg4  H5120 E128 F1536 top-8 S1 W4A16 int4 g128 (bf16 scales, zero point 8),
        8 prefill chunks of 512 + 248 decode tokens (N=4344)
  cfg5  H7168 E256 F2048 top-8 S0 fp8 e4m3fn 128x128, 8192 tokens, fixed-shape routing with
        a per-expert bias beta * ln(p_e), p_e ~ Zipf(1.2), beta chosen so the realised load is
        closest to Zipf(1.2) in KL, and 16 experts that receive no tokens

Derivation (seeded ``torch.Generator`` on the generation device, in this order): token
lengths, x ~ N(0,1), gate weight ~ N(0, 0.02), complexity predictor W1, W2 ~ N(0, 0.02)
with zero biases, then per expert (routed 0..E-1, then shared) Wg, Wu, Wd ~ N(0, 0.02)
drawn in fp32 and packed one expert at a time. cfg5's bias comes from a numpy generator
seeded with the same seed.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np
import torch

from . import _lib
from .quant import ExpertPacker, PackedExperts


@dataclass(frozen=True)
class LayerSpec:
    name: str
    hidden: int
    ffn: int
    num_experts: int
    top_k: int
    num_shared: int
    fmt: int
    act_dtype: torch.dtype
    fixed_shape_mode: bool = False
    zipf_s: float = 0.0
    zero_experts: int = 0
    zipf_beta: float = 1.0


SPECS = {
    "cfg1": LayerSpec("cfg1", 1024, 2816, 8, 2, 1, _lib.W_F32, torch.float32),
    "cfg2": LayerSpec("cfg2", 4096, 1408, 64, 6, 2, _lib.W_INT8, torch.bfloat16),
    "cfg3": LayerSpec("cfg3", 4096, 1408, 64, 6, 2, _lib.W_INT8, torch.bfloat16),
    "cfg4": LayerSpec("cfg4", 5120, 1536, 128, 8, 1, _lib.W_INT4, torch.bfloat16),
    # zipf_beta: the bias scale whose realised top-8 load is closest to Zipf(1.2) in KL
    # (zipf_beta_search over 0.50 .. 2.00 in steps of 0.05 on cfg5's logits; checked by
    # tests/test_workloads.py)
    "cfg5": LayerSpec("cfg5", 7168, 2048, 256, 8, 0, _lib.W_FP8, torch.bfloat16,
                      fixed_shape_mode=True, zipf_s=1.2, zero_experts=16, zipf_beta=1.0),
}


def seq_lengths(name: str, seed: int = 0) -> List[int]:
    """Sequence lengths of the packed batch of a configuration."""
    if name == "cfg1":
        g = torch.Generator().manual_seed(seed)
        return torch.randint(1, 257, (16,), generator=g).tolist()
    if name == "cfg2":
        return [1] * 64
    if name == "cfg3":
        # log-normal(6, 0.8) clipped to [16, 2048]; redraw the 32 lengths until the total is
        # within 512 of 16384 (the plain seed-0 draw gives 14,617)
        rng = np.random.default_rng(seed)
        while True:
            l = np.clip(np.round(rng.lognormal(6.0, 0.8, 32)), 16, 2048).astype(int)
            if abs(int(l.sum()) - 16384) <= 512:
                return l.tolist()
    if name == "cfg4":
        return [512] * 8 + [1] * 248
    if name == "cfg5":
        return [8192]
    raise KeyError(name)


def cu_seqlens(lengths: List[int]) -> torch.Tensor:
    return torch.tensor([0] + list(np.cumsum(lengths)), dtype=torch.int32)


@dataclass
class Workload:
    spec: LayerSpec
    lengths: List[int]
    x: torch.Tensor                       # [N, H] activations
    gate_weight: torch.Tensor             # [E, H] (fp32 cfg1, bf16 otherwise)
    pred: Optional[tuple]                 # (W1 [64,H], b1 [64], W2 [1,64], b2 [1]) fp32
    expert_bias: Optional[torch.Tensor]   # [E] fp32 (fixed-shape mode)
    experts: PackedExperts
    shared_expert_weight: Optional[torch.Tensor]
    meta: dict = field(default_factory=dict)

    @property
    def n_tokens(self) -> int:
        return int(self.x.shape[0])


def zipf_target(E: int, s: float, zero: int, seed: int) -> np.ndarray:
    """Target load share of each expert: p_e ~ rank_e^-s over a seeded permutation of the
    experts, 0 for the `zero` seeded tail experts, normalised over the others."""
    rng = np.random.default_rng(seed)
    order = rng.permutation(E)
    rank = np.empty(E, dtype=np.int64)
    rank[order] = np.arange(1, E + 1)
    p = rank.astype(np.float64) ** (-s)
    p[order[E - zero:]] = 0.0
    return p / p.sum()


def zipf_bias(E: int, s: float, zero: int, seed: int, beta: float = 1.0) -> np.ndarray:
    """expert_bias_e = beta * ln(p_e) with p_e ~ rank^-s over a seeded permutation; `zero`
    seeded tail experts get -30 so that they receive no tokens."""
    rng = np.random.default_rng(seed)
    order = rng.permutation(E)
    rank = np.empty(E, dtype=np.int64)
    rank[order] = np.arange(1, E + 1)
    p = rank.astype(np.float64) ** (-s)
    p /= p.sum()
    bias = (beta * np.log(p)).astype(np.float32)
    bias[order[E - zero:]] = -30.0
    return bias


def load_kl(counts, target: np.ndarray) -> float:
    """KL(realised || target) in nats of an expert-load histogram (slot counts per expert)
    against the target shares; experts with no load add nothing, load on an expert whose target
    is 0 gives inf."""
    c = np.asarray(counts, dtype=np.float64)
    q = c / c.sum()
    m = q > 0
    if np.any(target[m] <= 0):
        return float("inf")
    return float((q[m] * np.log(q[m] / target[m])).sum())


def zipf_beta_search(logits: torch.Tensor, spec: "LayerSpec", seed: int = 0,
                     grid=None) -> tuple:
    """The bias scale beta (on a grid, default 0.50 .. 2.00 in steps of 0.05) whose realised
    load — top-k of logits + zipf_bias(beta), as the fixed-shape router ranks them — is closest
    in KL to the Zipf(s) target. With top-k routing no expert can take more than one slot per
    token, so the heaviest Zipf shares are out of reach and the KL stays above 0. Returns
    (beta, kl)."""
    if grid is None:
        grid = [round(0.5 + 0.05 * i, 2) for i in range(31)]
    E, k = spec.num_experts, spec.top_k
    target = zipf_target(E, spec.zipf_s, spec.zero_experts, seed)
    best = None
    lg = logits.float()
    for beta in grid:
        b = torch.from_numpy(zipf_bias(E, spec.zipf_s, spec.zero_experts, seed, beta)).to(lg.device)
        idx = torch.topk(lg + b, k, dim=1).indices.reshape(-1).cpu().numpy()
        kl = load_kl(np.bincount(idx, minlength=E), target)
        if best is None or kl < best[1]:
            best = (beta, kl)
    return best


def make_workload(name, device="cpu", seed: int = 0, n_tokens: Optional[int] = None,
                  hidden: Optional[int] = None, ffn: Optional[int] = None,
                  num_experts: Optional[int] = None,
                  lengths: Optional[List[int]] = None) -> Workload:
    """Build a configuration's seeded inputs and packed layer on ``device``.

    ``name`` is a configuration name or a LayerSpec. n_tokens / hidden / ffn / num_experts
    shrink the configuration for CPU-checkable parity tests (same formats and routing
    modes, smaller shapes); ``lengths`` replaces the packed batch's sequence lengths.
    """
    base = name if isinstance(name, LayerSpec) else SPECS[name]
    name = base.name
    spec = LayerSpec(base.name, hidden or base.hidden, ffn or base.ffn,
                     num_experts or base.num_experts, min(base.top_k, num_experts or base.num_experts),
                     base.num_shared, base.fmt, base.act_dtype, base.fixed_shape_mode, base.zipf_s,
                     min(base.zero_experts, max(0, (num_experts or base.num_experts) - base.top_k)),
                     base.zipf_beta)
    dev = torch.device(device)
    if lengths is None:
        lengths = seq_lengths(name, seed)
    N = sum(lengths) if n_tokens is None else n_tokens
    if n_tokens is not None:
        lengths = [n_tokens]
    g = torch.Generator(device=dev).manual_seed(seed)
    H, Fd, E, S = spec.hidden, spec.ffn, spec.num_experts, spec.num_shared
    x = torch.randn(N, H, generator=g, device=dev).to(spec.act_dtype)
    gate_w = (torch.randn(E, H, generator=g, device=dev) * 0.02).to(spec.act_dtype)
    pred = None
    if not spec.fixed_shape_mode:
        W1 = torch.randn(64, H, generator=g, device=dev) * 0.02
        W2 = torch.randn(1, 64, generator=g, device=dev) * 0.02
        pred = (W1, torch.zeros(64, device=dev), W2, torch.zeros(1, device=dev))
    bias = None
    meta = {"seed": seed, "n_tokens": N}
    if spec.fixed_shape_mode and spec.zipf_s > 0:
        bias = torch.from_numpy(zipf_bias(E, spec.zipf_s, spec.zero_experts, seed,
                                          spec.zipf_beta)).to(dev)
        meta["zipf_s"] = spec.zipf_s
        meta["zipf_beta"] = spec.zipf_beta
        meta["zero_experts"] = spec.zero_experts
    pk = ExpertPacker(spec.fmt, E, S, H, Fd, dev)
    for i in range(E + S):
        wg = torch.randn(Fd, H, generator=g, device=dev) * 0.02
        wu = torch.randn(Fd, H, generator=g, device=dev) * 0.02
        wd = torch.randn(H, Fd, generator=g, device=dev) * 0.02
        pk.set(i, wg, wu, wd)
    sew = (torch.ones(S, device=dev) / S).to(spec.act_dtype) if S > 0 else None
    return Workload(spec, lengths, x, gate_w, pred, bias, pk.packed, sew, meta)


def router_state(w: Workload):
    """RouterState of a workload (YvStableMoEGate defaults: capacity_factor 1, min_capacity 4)."""
    from .functional import RouterState
    from .quant import pack_router
    act = _lib.ACT_BF16 if w.spec.act_dtype == torch.bfloat16 else _lib.ACT_F32
    W1 = w.pred[0] if w.pred is not None else None
    wr = pack_router(w.gate_weight, W1, act)
    b1 = w.pred[1].float().contiguous() if w.pred is not None else None
    w2 = w.pred[2].float().reshape(-1).contiguous() if w.pred is not None else None
    b2 = w.pred[3].float().reshape(-1).contiguous() if w.pred is not None else None
    return RouterState(w.spec.num_experts, w.spec.hidden, w.spec.top_k, w.spec.fixed_shape_mode,
                       not w.spec.fixed_shape_mode, 4, 1.0, wr, b1, w2, b2,
                       None if w.expert_bias is None else w.expert_bias.float().contiguous())


def mix_weights(w: Workload) -> Optional[torch.Tensor]:
    if w.shared_expert_weight is None:
        return None
    return torch.softmax(w.shared_expert_weight, dim=0).float().contiguous()


# ---------------------------------------------------------------- algorithmic work
def weight_bytes_per_expert(spec: LayerSpec) -> int:
    H, Fd = spec.hidden, spec.ffn
    if spec.fmt == _lib.W_INT8:
        return 3 * H * Fd + (2 * Fd + H) * 2
    if spec.fmt == _lib.W_INT4:
        return 3 * H * Fd // 2 + (2 * Fd * H // 128 + H * Fd // 128) * 2
    if spec.fmt == _lib.W_FP8:
        return 3 * H * Fd + (2 * (Fd // 128) * (H // 128) + (H // 128) * (Fd // 128)) * 4
    if spec.fmt == _lib.W_BF16:
        return 6 * H * Fd
    return 12 * H * Fd


def algorithmic_work(spec: LayerSpec, n_tokens: int, active_experts: int, skip: bool) -> dict:
    """FLOPs and HBM bytes of one forward (all N*k slots computed, as the reference does).

    bytes = weights of the active routed experts + shared experts + gate (+ predictor W1)
            + x + out (+ shared_out and skip when shared experts exist).
    """
    H, E, k, S = spec.hidden, spec.num_experts, spec.top_k, spec.num_shared
    act_b = 2 if spec.act_dtype == torch.bfloat16 else 4
    gate_b = 2 if spec.act_dtype == torch.bfloat16 else 4
    flops = 2 * n_tokens * H * E + 6 * H * spec.ffn * (n_tokens * k + n_tokens * S)
    pred_bytes = 0
    if not spec.fixed_shape_mode:
        flops += 2 * n_tokens * H * 64
        pred_bytes = 64 * H * 4
    wbytes = (active_experts + S) * weight_bytes_per_expert(spec)
    bytes_ = wbytes + E * H * gate_b + pred_bytes + 2 * n_tokens * H * act_b
    if S > 0:
        bytes_ += n_tokens * H * act_b * (2 if skip else 1)
    return {"flops": flops, "bytes": bytes_, "weight_bytes": wbytes}
