"""Routing on the GPU is bit-exact against the CPU oracle given identical fp32 logits.

Covers the configurations' (N, E, k) shapes with the capacity they see, fixed-shape mode with
a Zipf bias and zero-load experts, exact ties (tie rule: lower expert index; capacity keeps
the earlier token), all tokens on one expert, cap 0, N = 0 and 1, k = E and k = 1, and a large
N that spans many scan blocks. Everything goes through the C ABI (yvmoe_route).
"""
import numpy as np
import pytest
import torch

from pisceslx_amd import functional as yvf
from pisceslx_amd.workloads import zipf_bias

pytestmark = pytest.mark.gpu


def _router(E, k, fixed, bias=None):
    dummy = torch.zeros(1, device="cuda")
    return yvf.RouterState(E, 64, k, fixed, False, 4, 1.0, dummy, None, None, None,
                           None if bias is None else torch.from_numpy(bias).cuda())


def _check(oracle, logits, k, cap, bias=None):
    N, E = logits.shape
    fixed = cap < 0
    print(f"route N={N} E={E} k={k} cap={cap} fixed={fixed}", flush=True)
    st = _router(E, k, fixed, bias)
    g = yvf.route(torch.from_numpy(logits).cuda(), st, predictor=False,
                  capacity_override=-1 if fixed else cap)
    torch.cuda.synchronize()
    o = oracle.route(logits, k, cap, bias)
    assert np.array_equal(g.indices.cpu().numpy(), o.indices.astype(np.int64))
    assert np.array_equal(g.weights.cpu().numpy().view(np.uint32), o.weights.view(np.uint32))
    assert np.array_equal(g.counts.cpu().numpy(), o.counts)
    assert np.array_equal(g.offsets.cpu().numpy(), o.offsets)
    assert np.array_equal(g.perm.cpu().numpy(), o.perm)
    assert np.array_equal(g.pos.cpu().numpy(), o.pos)
    assert int(g.capacity.item()) == (cap if not fixed else -1)


@pytest.mark.parametrize("N,E,k,cap", [
    (2052, 8, 2, 320),      # cfg1 shape
    (64, 64, 6, 4),         # cfg2 decode, cap = min_capacity
    (16384, 64, 6, 320),    # cfg3 prefill
    (4344, 128, 8, 42),     # cfg4
    (65536, 8, 2, 9000),    # many scan blocks
    (1, 8, 2, 4),
    (7, 5, 5, 2),           # k = E
    (300, 16, 1, 10),       # k = 1
    (100, 256, 16, 3),      # max E and k
])
def test_route_bit_exact(cuda, oracle, N, E, k, cap):
    rng = np.random.default_rng(N * 7 + E)
    logits = (rng.standard_normal((N, E)) * 1.7).astype(np.float32)
    _check(oracle, logits, k, cap)


def test_route_fixed_mode_zipf(cuda, oracle):
    rng = np.random.default_rng(11)
    E, k, N = 256, 8, 8192
    bias = zipf_bias(E, 1.2, 16, 0)
    logits = (rng.standard_normal((N, E)) * 1.7).astype(np.float32)
    _check(oracle, logits, k, -1, bias)


@pytest.mark.parametrize("E,k,cap", [(8, 2, 5), (64, 6, 3), (256, 8, 2)])
def test_route_exact_ties(cuda, oracle, E, k, cap):
    rng = np.random.default_rng(E + k)
    logits = rng.integers(-1, 2, size=(777, E)).astype(np.float32)
    _check(oracle, logits, k, cap)


def test_route_all_to_one_expert(cuda, oracle):
    rng = np.random.default_rng(5)
    N, E, k = 1000, 16, 2
    logits = (rng.standard_normal((N, E)) * 0.1).astype(np.float32)
    logits[:, 3] += 20.0
    for cap in (0, 1, 17, 999, 1000):
        _check(oracle, logits, k, cap)


def test_route_empty_batch(cuda, oracle):
    st = _router(8, 2, False)
    g = yvf.route(torch.zeros(0, 8, device="cuda"), st, predictor=False, capacity_override=4)
    torch.cuda.synchronize()
    assert g.counts.cpu().tolist() == [0] * 8
    assert g.offsets.cpu().tolist() == [0] * 9


def test_route_deterministic(cuda, oracle):
    rng = np.random.default_rng(9)
    logits = torch.from_numpy((rng.standard_normal((20000, 64)) * 1.7).astype(np.float32)).cuda()
    st = _router(64, 6, False)
    a = yvf.route(logits, st, predictor=False, capacity_override=300)
    b = yvf.route(logits, st, predictor=False, capacity_override=300)
    for x, y in ((a.perm, b.perm), (a.weights, b.weights), (a.pos, b.pos)):
        assert torch.equal(x, y)


@pytest.mark.parametrize("N,E,k,cap", [
    (256, 64, 6, 3),        # largest batch of the single-work-group path
    (257, 64, 6, 3),        # smallest batch of the multi-block path
    (200, 8, 2, 5),
    (129, 256, 16, 1),
    (64, 64, 6, 0),
])
def test_route_small_batch_boundary(cuda, oracle, N, E, k, cap):
    rng = np.random.default_rng(N * 13 + E)
    logits = (rng.standard_normal((N, E)) * 1.7).astype(np.float32)
    _check(oracle, logits, k, cap)


@pytest.mark.parametrize("E,k,cap", [(8, 2, 5), (64, 6, 3), (256, 8, 2)])
def test_route_small_batch_ties(cuda, oracle, E, k, cap):
    rng = np.random.default_rng(E * 3 + k)
    logits = rng.integers(-1, 2, size=(200, E)).astype(np.float32)
    _check(oracle, logits, k, cap)


def test_route_small_batch_one_expert_and_fixed(cuda, oracle):
    rng = np.random.default_rng(6)
    N, E, k = 200, 16, 2
    logits = (rng.standard_normal((N, E)) * 0.1).astype(np.float32)
    logits[:, 3] += 20.0
    for cap in (0, 1, 17, 199, 200):
        _check(oracle, logits, k, cap)
    E, k, N = 256, 8, 128
    bias = zipf_bias(E, 1.2, 16, 0)
    logits = (rng.standard_normal((N, E)) * 1.7).astype(np.float32)
    _check(oracle, logits, k, -1, bias)
