"""Pins the CPU routing oracle (oracle/route_oracle.c) before it is trusted as the checker.

Checks: yv_expf against libm in float64 (<= 2 ulp); the softmax against float64 (<= 4 ulp
relative); top-k against brute force over all subsets, with forced ties; the whole routing
against a restatement of YvStableMoEGate (model/moe/gate.py:1147-1241) that uses torch's own
softmax / topk / bincount — every disagreement must sit on a float64 near-tie; the capacity
formula against the reference's Python expression (gate.py:1117-1120, :1173-1176); the
capacity invariants of tools/test/test_moe_routing_contract.py:84-112; and the permutation
against numpy's stable argsort (opss/infer/fused_moe.py:87-95).
"""
import itertools
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F


def ulp_diff(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    ai = a.astype(np.float32).view(np.int32).astype(np.int64)
    bi = b.astype(np.float32).view(np.int32).astype(np.int64)
    return np.abs(ai - bi)


def test_expf_against_libm(oracle):
    x = np.linspace(-86.0, 0.0, 400_001, dtype=np.float32)
    x = np.concatenate([x, np.array([0.0, -1e-30, -1e-7, -0.34657359, -0.34657360, -85.99],
                                    dtype=np.float32)])
    got = oracle.expf(x)
    ref = np.exp(x.astype(np.float64)).astype(np.float32)
    assert ulp_diff(got, ref).max() <= 2
    assert oracle.expf(np.array([-86.5, -1000.0, -np.inf], dtype=np.float32)).tolist() == [0, 0, 0]
    assert oracle.expf(np.array([0.0], dtype=np.float32))[0] == 1.0


def test_softmax_against_float64(oracle):
    rng = np.random.default_rng(1)
    for E in (8, 16, 64, 128, 256, 5):
        z = (rng.standard_normal((64, E)) * 3).astype(np.float32)
        p = oracle.softmax_rows(z)
        # float64 exp and sum of the same fp32-rounded differences z - max
        d = (z - z.max(1, keepdims=True)).astype(np.float64)
        ref = np.exp(d)
        ref /= ref.sum(1, keepdims=True)
        rel = np.abs(p - ref) / ref
        assert rel.max() < 4 * 2.0 ** -23, (E, rel.max())


def brute_topk(p: np.ndarray, k: int):
    """The unique k-subset whose members all beat all non-members under (p desc, e asc)."""
    E = len(p)
    beats = lambda a, b: p[a] > p[b] or (p[a] == p[b] and a < b)
    found = []
    for sub in itertools.combinations(range(E), k):
        rest = [e for e in range(E) if e not in sub]
        if all(beats(a, b) for a in sub for b in rest):
            found.append(sub)
    assert len(found) == 1
    return sorted(found[0], key=lambda e: (-p[e], e))


@pytest.mark.parametrize("E,k", [(6, 2), (8, 3), (7, 7), (9, 1)])
def test_topk_brute_force_with_ties(oracle, E, k):
    rng = np.random.default_rng(E * 10 + k)
    # quantized logits force exact ties in p
    z = rng.integers(-2, 3, size=(200, E)).astype(np.float32)
    r = oracle.route(z, k, -1)
    p = oracle.softmax_rows(z)
    for t in range(z.shape[0]):
        want = brute_topk(p[t], k)
        assert list(r.indices[t]) == want
        assert np.array_equal(r.topp[t], p[t][want])


def torch_gate_route(logits: np.ndarray, k: int, cap: int, bias=None):
    """YvStableMoEGate's routing written with the reference's torch calls (gate.py:1147-1241)."""
    z = torch.from_numpy(logits.copy())
    if bias is not None:
        z = z + torch.from_numpy(bias)
    scores = F.softmax(z, dim=-1)
    top_scores, top_idx = torch.topk(scores, k, dim=-1)
    weights = F.softmax(top_scores, dim=-1, dtype=torch.float32).type_as(top_scores)
    if cap < 0:
        return weights.numpy(), top_idx.numpy(), scores.numpy()
    E = z.shape[1]
    allowed = torch.ones_like(top_idx, dtype=torch.bool)
    counts = torch.bincount(top_idx.flatten(), minlength=E)
    for e in (counts > cap).nonzero().squeeze(-1).tolist():
        slots = top_idx == e
        positions = slots.any(dim=-1).nonzero(as_tuple=True)[0]
        surplus = int(positions.numel()) - cap
        if surplus <= 0:
            continue
        ranked = torch.topk(scores[positions, e], surplus, largest=False)
        dropped = positions[ranked.indices]
        allowed[dropped] = allowed[dropped] & ~slots[dropped]
    weights = weights * allowed.to(weights.dtype)
    total = weights.sum(dim=-1, keepdim=True)
    weights = weights * (total > 0).to(weights.dtype) / total.clamp(min=1e-8)
    return weights.numpy(), top_idx.numpy(), scores.numpy()


def near_tie_tokens(logits: np.ndarray, k: int, bias=None, rel=1e-6):
    z = logits.astype(np.float64) + (0 if bias is None else bias.astype(np.float64))
    p = np.exp(z - z.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    s = -np.sort(-p, axis=1)
    gap = (s[:, k - 1] - s[:, k]) / s[:, k - 1] if k < z.shape[1] else np.ones(len(z))
    return set(np.nonzero(gap < rel)[0].tolist())


@pytest.mark.parametrize("N,E,k,cap", [(2052, 8, 2, 320), (64, 64, 6, 4), (4000, 64, 6, 300),
                                       (1200, 128, 8, 60), (512, 256, 8, -1)])
def test_routing_matches_torch_restatement(oracle, N, E, k, cap):
    rng = np.random.default_rng(N + E)
    logits = (rng.standard_normal((N, E)) * 1.7).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.5).astype(np.float32) if cap < 0 else None
    r = oracle.route(logits, k, cap, bias)
    w_t, idx_t, scores_t = torch_gate_route(logits, k, cap, bias)
    ties = near_tie_tokens(logits, k, bias)
    bad = np.nonzero((r.indices != idx_t).any(1))[0]
    assert set(bad.tolist()) <= ties
    ok = np.setdiff1d(np.arange(N), bad)
    if cap >= 0:
        # a capacity decision can also flip on a near tie of p across tokens; count them
        flips = np.nonzero(np.abs(r.weights[ok] - w_t[ok]).max(1) > 1e-6)[0]
        assert len(flips) <= max(1, N // 1000)
        ok = np.setdiff1d(ok, ok[flips])
    np.testing.assert_allclose(r.weights[ok], w_t[ok], rtol=0, atol=1e-6)
    assert (r.indices[ok] == idx_t[ok]).all()


def test_capacity_formula_matches_reference_expression(oracle):
    rng = np.random.default_rng(3)
    for _ in range(20000):
        N = int(rng.integers(0, 40000))
        E = int(rng.choice([8, 64, 128, 256]))
        avg = float(np.float32(rng.uniform(-0.1, 1.1)))
        mc = int(rng.integers(0, 8))
        dynamic_factor = 0.5 + 1.5 * avg                       # gate.py:1119
        cf = max(0.5, min(2.0, dynamic_factor))                # gate.py:1120
        want = max(int(N * cf / E), mc)                        # gate.py:1173-1176
        assert oracle.capacity(avg, N, E, mc) == want


def test_capacity_contract_invariants(oracle):
    """tools/test/test_moe_routing_contract.py:84-112 with every token preferring expert 0."""
    rng = np.random.default_rng(4)
    T, E, k = 24, 4, 2
    x = rng.standard_normal((T, 32)).astype(np.float32)
    W = np.zeros((E, 32), dtype=np.float32)
    W[0] = 1.0
    logits = x @ W.T
    for cap in (1, 5, 6, 12, 24, 30):
        r = oracle.route(logits, k, cap)
        served = int(((r.indices == 0) & (r.weights > 0)).sum())
        collapsed = int((r.indices == 0).any(1).sum())
        assert served <= cap
        if collapsed > cap:
            assert served == cap
        else:
            assert served == collapsed
        tot = r.weights.sum(1)
        kept = tot > 0
        np.testing.assert_allclose(tot[kept], 1.0, atol=1e-5)
        assert (r.weights >= 0).all() and ((tot <= 1 + 1e-5) | (tot == 0)).all()


def test_capacity_drop_order_and_ties(oracle):
    """Dropped tokens are the lowest p on the expert; equal p drops the later token."""
    N, E, k = 10, 3, 1
    logits = np.zeros((N, E), dtype=np.float32)
    logits[:, 0] = 5.0
    logits[[2, 7], 0] = 4.0   # lowest p on expert 0, tied
    logits[5, 0] = 4.5
    r = oracle.route(logits, k, 8)
    dropped = sorted(np.nonzero(r.allowed[:, 0] == 0)[0].tolist())
    assert dropped == [2, 7]
    r = oracle.route(logits, k, 7)
    dropped = sorted(np.nonzero(r.allowed[:, 0] == 0)[0].tolist())
    assert dropped == [2, 5, 7]
    r = oracle.route(logits, k, 9)   # one of the tied pair goes: the later token
    dropped = sorted(np.nonzero(r.allowed[:, 0] == 0)[0].tolist())
    assert dropped == [7]
    assert (r.weights[r.allowed[:, 0] == 0] == 0).all()


def test_permutation_is_stable_argsort(oracle):
    rng = np.random.default_rng(5)
    for N, E, k in ((1, 4, 2), (37, 8, 2), (500, 64, 6), (300, 256, 8)):
        logits = rng.standard_normal((N, E)).astype(np.float32)
        r = oracle.route(logits, k, -1)
        flat = r.indices.reshape(-1)
        perm = np.argsort(flat, kind="stable")
        assert np.array_equal(r.perm, perm)
        assert np.array_equal(r.counts, np.bincount(flat, minlength=E))
        assert np.array_equal(r.offsets, np.concatenate([[0], np.cumsum(r.counts)]))
        assert np.array_equal(r.pos[r.perm], np.arange(N * k))
        for t in range(N):
            assert len(set(r.indices[t].tolist())) == k


def test_double_softmax_closed_form(oracle):
    rng = np.random.default_rng(6)
    logits = rng.standard_normal((100, 16)).astype(np.float32)
    r = oracle.route(logits, 4, -1)
    ts = r.topp.astype(np.float64)
    ref = np.exp(ts - ts[:, :1])
    ref /= ref.sum(1, keepdims=True)
    np.testing.assert_allclose(r.weights, ref, rtol=4e-7, atol=0)
    assert (np.diff(r.topp, axis=1) <= 0).all()


def test_empty_batch(oracle):
    r = oracle.route(np.zeros((0, 8), dtype=np.float32), 2, 4)
    assert r.counts.tolist() == [0] * 8 and r.offsets.tolist() == [0] * 9
