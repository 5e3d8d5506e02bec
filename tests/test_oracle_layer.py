"""Pins the oracle's expert math and combine (oracle/moe_oracle.py: linear, swiglu,
layer_forward, complexity_scores, layer_capacity) against what the mathematics fixes,
independently of the oracle's own formulas:

* SwiGLU known answers: one-hot inputs pick weight columns, so y follows in closed form from
  the chosen columns (a transposed operand, a gate/up swap or a wrong rounding point fails);
  a permutation down-projection checks the orientation of Wd.
* correctly rounded linear: against exact rational arithmetic on small integer-valued
  operands, and its single rounding against a double-rounded alternative.
* the whole layer against an independent float64 dense formulation: a dense [N, E] routing
  matrix built from the routing's (index, weight) pairs, every expert applied to every token,
  mixture weights softmax(shared_expert_weight) (= the mean for the default ones/S), and the
  skip residual (model/moe/layer.py:741-753, :812-865, :867-963; opss/infer/fused_moe.py:54-123).
* the skip residual is exactly 0.1 * skip on top of the same output (fp32 layer); the token
  subset option reproduces the rows of the full forward.
* complexity predictor and dynamic capacity from constructed predictor weights
  (model/moe/gate.py:1096-1120, :1172-1176).
"""
import math
from fractions import Fraction

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import moe_oracle as mo


def _bf16(v: float) -> float:
    return float(torch.tensor(v, dtype=torch.float64).to(torch.bfloat16).double())


def _silu(v: float) -> float:
    return v / (1.0 + math.exp(-v))


def test_swiglu_one_hot_known_answer():
    torch.manual_seed(0)
    H, Fd = 8, 8
    a = (torch.randn(Fd) * 2).to(torch.bfloat16)   # gate column
    b = (torch.randn(Fd) * 2).to(torch.bfloat16)   # up column
    i = 5
    wg = torch.zeros(Fd, H, dtype=torch.bfloat16)
    wu = torch.zeros(Fd, H, dtype=torch.bfloat16)
    wg[:, i] = a
    wu[:, i] = b
    wg[:, 2] = 7.0                                 # other columns must not leak in
    wu[:, 3] = -3.0
    perm = torch.tensor([3, 0, 7, 1, 6, 2, 5, 4])
    wd = torch.zeros(H, Fd, dtype=torch.bfloat16)
    wd[torch.arange(H), perm] = 1.0                # y[r] = h[perm[r]]
    x = torch.zeros(1, H, dtype=torch.bfloat16)
    x[0, i] = 1.0
    y = mo.swiglu(x, wg, wu, wd)[0]
    for r in range(H):
        f = int(perm[r])
        g, u = float(a[f]), float(b[f])
        # rounding points of the reference bf16 chain: silu(g) -> bf16, silu * u -> bf16
        want = _bf16(_bf16(_silu(g)) * u)
        assert float(y[r]) == want, (r, float(y[r]), want)


def test_linear_is_correctly_rounded():
    rng = np.random.default_rng(1)
    # integer-valued operands: the exact sum is an integer, its rounding is known exactly
    x = torch.from_numpy(rng.integers(-40, 41, size=(3, 64)).astype(np.float32)).to(torch.bfloat16)
    w = torch.from_numpy(rng.integers(-40, 41, size=(5, 64)).astype(np.float32)).to(torch.bfloat16)
    got = mo.linear(x, w)
    for i in range(3):
        for j in range(5):
            exact = sum(Fraction(int(x[i, q])) * Fraction(int(w[j, q])) for q in range(64))
            assert float(got[i, j]) == _bf16(float(exact))
    # one rounding: a sum that lands between bf16 neighbours rounds to nearest, not through an
    # intermediate fp32 rounding of partial sums
    x = torch.tensor([[256.0, 1.0, 1.0]], dtype=torch.bfloat16)
    w = torch.tensor([[1.0, 1.0, 0.5]], dtype=torch.bfloat16)
    assert float(mo.linear(x, w)[0, 0]) == _bf16(257.5)  # = 258 (bf16 spacing 2 above 256)


def _dense_layer_f64(x, params, routing, skip):
    """Independent float64 statement of routed + shared + 0.1 * skip."""
    N, H = x.shape
    E, S, k = params.num_experts, params.num_shared, params.top_k
    Rw = np.zeros((N, E))
    for t in range(N):
        for j in range(k):
            Rw[t, routing.indices[t, j]] += routing.weights[t, j]
    xd = x.double()
    out = torch.zeros(N, H, dtype=torch.float64)
    for e in range(E):
        wg, wu, wd = (m.double() for m in params.expert(e))
        ye = (F.silu(xd @ wg.t()) * (xd @ wu.t())) @ wd.t()
        out += torch.from_numpy(Rw[:, e:e + 1]) * ye
    if S > 0:
        mix = torch.softmax(params.mix_param.double(), dim=0)
        for s in range(S):
            wg, wu, wd = (m.double() for m in params.expert(E + s))
            out += mix[s] * ((F.silu(xd @ wg.t()) * (xd @ wu.t())) @ wd.t())
        if skip is not None:
            out += 0.1 * skip.double()
    return out


def _small_params(H=32, Fd=48, E=6, S=2, k=3, seed=0):
    g = torch.Generator().manual_seed(seed)
    mats = [tuple(torch.randn(*shp, generator=g) * 0.2 for shp in ((Fd, H), (Fd, H), (H, Fd)))
            for _ in range(E + S)]
    return mo.LayerParams(
        hidden=H, ffn=Fd, num_experts=E, num_shared=S, top_k=k,
        gate_weight=torch.randn(E, H, generator=g) * 0.5, pred=None, bias=None,
        fixed_shape_mode=True, dynamic_capacity=False, capacity_factor=1.0, min_capacity=1,
        mix_param=torch.ones(S) / S if S else None, expert_fn=lambda i: mats[i])


@pytest.mark.parametrize("cap", [-1, 2])
def test_layer_forward_matches_dense_f64(cap):
    p = _small_params()
    if cap >= 0:
        p.fixed_shape_mode = False
    g = torch.Generator().manual_seed(7)
    x = torch.randn(11, p.hidden, generator=g)
    skip = torch.randn(11, p.hidden, generator=g)
    o = mo.layer_forward(x, p, cap=cap, skip=skip)
    r = o["routing"]
    if cap >= 0:
        assert int(r.allowed.size - r.allowed.sum()) > 0  # the trim is exercised
    want = _dense_layer_f64(x, p, r, skip)
    assert float((o["out"].double() - want).abs().max()) < 2e-5
    # S = 2 with the default ones/S parameter: the mixture is the mean of the shared experts
    shared = torch.zeros_like(want)
    for s in range(p.num_shared):
        wg, wu, wd = (m.double() for m in p.expert(p.num_experts + s))
        shared += ((F.silu(x.double() @ wg.t()) * (x.double() @ wu.t())) @ wd.t()) / p.num_shared
    assert float((o["shared"].double() - shared).abs().max()) < 2e-5


def test_skip_residual_and_token_subset():
    p = _small_params(seed=3)
    g = torch.Generator().manual_seed(9)
    x = torch.randn(9, p.hidden, generator=g)
    skip = torch.randn(9, p.hidden, generator=g)
    a = mo.layer_forward(x, p)["out"]
    b = mo.layer_forward(x, p, skip=skip)["out"]
    assert float(((b - a).double() - 0.1 * skip.double()).abs().max()) < 1e-6
    wrong = mo.layer_forward(x, p, skip=skip[:5])["out"]  # shape mismatch: no residual
    assert torch.equal(wrong, a)
    tok = np.array([1, 4, 8])
    c = mo.layer_forward(x, p, tokens=tok)["out"]
    assert torch.equal(c[tok], a[tok])


def test_complexity_and_dynamic_capacity_closed_form():
    H, E, N = 16, 8, 40
    W1 = torch.zeros(64, H)
    b1 = torch.full((64,), 0.25)
    b1[::2] = -1.0                      # relu drops half of the hidden units
    W2 = torch.full((1, 64), 0.5)
    b2 = torch.tensor([-3.0])
    x = torch.randn(N, H)
    s = mo.complexity_scores(x, (W1, b1, W2, b2))
    z = 32 * 0.5 * 0.25 - 3.0           # w2 . relu(b1) + b2
    want = 1.0 / (1.0 + math.exp(-z))
    assert torch.allclose(s.double(), torch.full((N,), want, dtype=torch.float64), atol=1e-7)
    p = _small_params(H=H, E=E)
    p.pred = (W1, b1, W2, b2)
    p.dynamic_capacity = True
    p.fixed_shape_mode = False
    p.min_capacity = 1
    cf = min(2.0, max(0.5, 0.5 + 1.5 * want))
    assert mo.layer_capacity(p, x) == max(int(N * cf / E), 1)
    p.min_capacity = 99
    assert mo.layer_capacity(p, x) == 99
