"""The dispatch operator (yvmoe_dispatch, PiscesLxFusedMoEDispatch) on the GPU against the CPU
oracle's dispatch (oracle/moe_oracle.py dispatch_forward), given the same external routing:

* counts, offsets and the expert outputs in expert-sorted order (stable by (token, slot))
  bit for bit in their order, the outputs within the layer tolerance;
* every weight format, decode-sized batches (streaming GEMMs) and prefill-sized ones (LDS-
  tiled GEMMs), fp32 and bf16 routing weights, zero-weight slots, experts with no slots, the
  same expert twice in one token, indices outside [0, E) (counted, never read through, the
  module raises);
* a routing from another router: the layer's own routing dispatched equals the layer's output
  (no shared experts), bit for bit;
* the module mirror: nn.ModuleList of SwiGLU experts, the size check (ValueError), collect_stats.
"""
import numpy as np
import pytest
import torch
import torch.nn as nn

from pisceslx_amd import _lib
from pisceslx_amd import functional as yvf
from pisceslx_amd.dispatch import PiscesLxFusedMoEDispatch, PiscesLxFusedMoe
from pisceslx_amd.workloads import make_workload, mix_weights, router_state

from helpers import check_close, check_ulps, oracle_params

pytestmark = pytest.mark.gpu


def _routing(N, k, E, seed, zero_frac=0.1, skew=False):
    rng = np.random.default_rng(seed)
    if skew:
        p = 1.0 / np.arange(1, E + 1) ** 1.2
        idx = rng.choice(E, size=(N, k), p=p / p.sum())
    else:
        idx = rng.integers(0, E, size=(N, k))
    w = rng.random((N, k))
    w[rng.random((N, k)) < zero_frac] = 0.0
    # weights of a token sum to 1 as a router's do (softmax, renormalised after a trim): the
    # output is then a convex combination of expert outputs, at their scale
    w = w / np.maximum(w.sum(axis=1, keepdims=True), 1e-12)
    return idx.astype(np.int64), w.astype(np.float32)


def _check_dispatch(oracle, w, idx, wts, label, tokens=None, weight_dtype=torch.float32):
    dev = w.x.device
    N = w.x.shape[0]
    E = w.spec.num_experts
    print(f"dispatch {label}", flush=True)
    idx_t = torch.from_numpy(idx).to(dev)
    w_t = torch.from_numpy(wts).to(weight_dtype).to(dev)
    out, counts, offsets, invalid, y = yvf.dispatch(w.x, w_t, idx_t, w.experts, want_expert_outputs=True)
    torch.cuda.synchronize()
    params = oracle_params(w)
    wref = w_t.float().cpu().numpy()
    d = oracle.dispatch_forward(w.x.cpu(), wref, idx, E, params.expert, tokens=tokens)
    assert np.array_equal(counts.cpu().numpy(), d.counts)
    assert np.array_equal(offsets.cpu().numpy(), d.offsets)
    assert int(invalid.item()) == d.invalid
    got, want = out.cpu(), d.out
    if tokens is not None:
        got, want = got[tokens], want[tokens]
        rows = np.nonzero(np.isin(d.perm // idx.shape[1], tokens))[0]
        gy, wy = y.cpu()[torch.from_numpy(rows)], d.Y[torch.from_numpy(rows)].to(w.x.dtype)
    else:
        V = len(d.perm)
        gy, wy = y.cpu()[:V], d.Y.to(w.x.dtype)
    if w.x.dtype == torch.bfloat16:
        check_ulps(gy, wy, f"dispatch {label} expert outputs")
    else:
        check_close(gy, wy, f"dispatch {label} expert outputs")
    check_close(got, want, f"dispatch {label}")
    return out


@pytest.mark.parametrize("name,kw,k", [
    ("cfg1", {"n_tokens": 300}, 2),
    ("cfg2", {}, 6),
    ("cfg2", {"n_tokens": 700}, 6),
    ("cfg4", {"n_tokens": 96}, 8),
    ("cfg5", {"n_tokens": 200, "num_experts": 32}, 8),
    ("cfg5", {"n_tokens": 64, "num_experts": 32}, 8),   # fp8 weights on the streaming form
    ("cfg5", {"n_tokens": 200, "num_experts": 32}, 12),  # the combine's second 8-slot chunk
    ("cfg5", {"n_tokens": 64, "num_experts": 32}, 16),   # the operator's largest k
    ("cfg2", {"n_tokens": 100}, 1),
])
def test_dispatch_matches_oracle(cuda, oracle, name, kw, k):
    w = make_workload(name, device=cuda, **kw)
    idx, wts = _routing(w.x.shape[0], k, w.spec.num_experts, seed=11)
    _check_dispatch(oracle, w, idx, wts, f"{name} N={w.x.shape[0]} k={k}")


def test_dispatch_prefill_tiled_bf16_weights_sampled(cuda, oracle):
    """A prefill-sized batch (LDS-tiled GEMMs) with skewed external routing, bf16 routing
    weights, some experts empty; checked on sampled tokens."""
    w = make_workload("cfg3", device=cuda, n_tokens=4096)
    N, E = w.x.shape[0], w.spec.num_experts
    idx, wts = _routing(N, 6, E, seed=12, skew=True)
    idx[idx >= E - 3] = 0  # the last three experts receive nothing
    rng = np.random.default_rng(3)
    tokens = np.sort(rng.choice(N, 64, replace=False))
    _check_dispatch(oracle, w, idx, wts, "cfg3 N=4096 k=6 skewed bf16 weights", tokens=tokens,
                    weight_dtype=torch.bfloat16)


def test_dispatch_duplicates_and_invalid_indices(cuda, oracle):
    w = make_workload("cfg2", device=cuda, n_tokens=40)
    N, E = 40, w.spec.num_experts
    idx, wts = _routing(N, 4, E, seed=13)
    idx[0] = [5, 5, 5, 5]
    idx[1, 2] = E
    idx[2, 0] = -7
    idx[3] = [E + 1, -1, 2 * E, E]  # a token with no valid slot: output zero
    wts[4] = 0.0
    out = _check_dispatch(oracle, w, idx, wts, "cfg2 N=40 duplicates / invalid indices")
    assert torch.count_nonzero(out[3]) == 0 and torch.count_nonzero(out[4]) == 0
    m = PiscesLxFusedMoEDispatch(E, 4).eval()
    with pytest.raises(RuntimeError, match="outside"):
        m(w.x, torch.from_numpy(wts).to(cuda), torch.from_numpy(idx).to(cuda), w.experts)
    m.check_indices = False
    got = m(w.x, torch.from_numpy(wts).to(cuda), torch.from_numpy(idx).to(cuda), w.experts)
    assert torch.equal(got, out)


def test_module_one_dimensional_indices(cuda, oracle):
    """expert_indices of shape [N] (one assignment per token, fused_moe.py:72-76) with routing
    weights of shape [N], through the module mirror."""
    w = make_workload("cfg2", device=cuda, n_tokens=90)
    N, E = 90, w.spec.num_experts
    idx, wts = _routing(N, 1, E, seed=15)
    m = PiscesLxFusedMoEDispatch(E, 1).eval()
    out = m(w.x, torch.from_numpy(wts.reshape(-1)).to(cuda), torch.from_numpy(idx.reshape(-1)).to(cuda),
            w.experts)
    torch.cuda.synchronize()
    assert out.shape == w.x.shape
    d = oracle.dispatch_forward(w.x.cpu(), wts, idx, E, oracle_params(w).expert)
    check_close(out, d.out, "dispatch module 1-D indices cfg2 N=90")


def test_dispatch_of_layer_routing_equals_layer(cuda):
    """Routing from the layer's own router, dispatched: the layer's output bit for bit (cfg5
    shape, no shared experts, so the layer output is the routed combine)."""
    w = make_workload("cfg5", device=cuda, n_tokens=300, num_experts=32)
    st, mix = router_state(w), mix_weights(w)
    out, _, routing = yvf.moe_forward(w.x, st, w.experts, mix, None)
    d = PiscesLxFusedMoe.fused_moe_dispatch(w.x, routing.weights, routing.indices, w.experts,
                                            w.spec.num_experts, w.spec.top_k)
    torch.cuda.synchronize()
    assert torch.equal(d, out)


class _SwiGLU(nn.Module):
    def __init__(self, H, F, dtype, device):
        super().__init__()
        self.gate_proj = nn.Linear(H, F, bias=False, device=device, dtype=dtype)
        self.up_proj = nn.Linear(H, F, bias=False, device=device, dtype=dtype)
        self.down_proj = nn.Linear(F, H, bias=False, device=device, dtype=dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_module_with_expert_modules(cuda, oracle, dtype):
    """The reference's call form: nn.ModuleList of SwiGLU experts (packed once, repacked when a
    weight changes), [N, k] routing, collect_stats."""
    torch.manual_seed(0)
    E, H, F, N, k = 6, 256, 384, 50, 2
    experts = nn.ModuleList([_SwiGLU(H, F, dtype, cuda) for _ in range(E)]).eval()
    x = torch.randn(N, H, device=cuda).to(dtype)
    idx, wts = _routing(N, k, E, seed=14)
    idx[idx == 5] = 4  # expert 5 unused
    idx_t, w_t = torch.from_numpy(idx).to(cuda), torch.from_numpy(wts).to(cuda)
    m = PiscesLxFusedMoEDispatch(E, k).eval()
    out, stats = m(x, w_t, idx_t, experts, collect_stats=True)
    fn = lambda e: tuple(getattr(experts[e], n).weight.detach().float().cpu()
                         for n in ("gate_proj", "up_proj", "down_proj"))
    d = oracle.dispatch_forward(x.cpu(), wts, idx, E, fn)
    check_close(out, d.out, f"dispatch module list {dtype}")
    active = [e for e in range(E) if d.counts[e] > 0]
    assert len(stats) == len(active) == 5
    for s, e in zip(stats, active):
        ye = d.Y[int(d.offsets[e]):int(d.offsets[e + 1])].to(dtype)
        torch.testing.assert_close(s.float().cpu(), ye.float().mean(0), atol=2e-2 if dtype == torch.bfloat16 else 1e-4,
                                   rtol=0)
    # a changed weight is picked up (repacked), and the size check raises like the reference
    with torch.no_grad():
        experts[1].down_proj.weight.mul_(2.0)
    out2 = m(x, w_t, idx_t, experts)
    d2 = oracle.dispatch_forward(x.cpu(), wts, idx, E, fn)
    check_close(out2, d2.out, f"dispatch module list {dtype} after a weight change")
    with pytest.raises(ValueError, match="assignments cannot come from"):
        m(x, w_t, idx_t.reshape(-1)[:-1], experts)


def test_dispatch_empty_batch(cuda):
    w = make_workload("cfg2", device=cuda, n_tokens=8)
    E = w.spec.num_experts
    x = w.x[:0]
    out, counts, offsets, invalid, _ = yvf.dispatch(
        x, torch.empty(0, 6, device=cuda), torch.empty(0, 6, dtype=torch.int64, device=cuda), w.experts)
    torch.cuda.synchronize()
    assert out.shape == (0, w.spec.hidden)
    assert counts.cpu().tolist() == [0] * E and offsets.cpu().tolist() == [0] * (E + 1)
    assert int(invalid.item()) == 0


def test_expert_ffn_with_a_fresh_workspace(cuda, oracle):
    """yvmoe_expert_ffn reads only the routing it is given: a routing computed in one
    workspace and the FFN run in another (never written before) give the same rows."""
    w = make_workload("cfg3", device=cuda, n_tokens=600)
    st = router_state(w)
    ws_a = torch.empty(yvf.workspace_bytes(600, _lib.ACT_BF16, st, w.experts), dtype=torch.uint8,
                       device=cuda)
    _, _, routing = yvf.moe_forward(w.x, st, w.experts, mix_weights(w), None, workspace=ws_a)
    ya = yvf.expert_ffn(w.x, w.experts, routing, w.spec.top_k, workspace=ws_a)
    ws_b = torch.full_like(ws_a, 0xA5)
    yb = yvf.expert_ffn(w.x, w.experts, routing, w.spec.top_k, workspace=ws_b)
    torch.cuda.synchronize()
    assert torch.equal(ya, yb)
