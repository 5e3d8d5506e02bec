"""Pins the YvMoEGate oracle (oracle/moegate_oracle.py) against what the mathematics fixes,
independently of the oracle's own formulas:

* top-k with ties to the lower index, and torch.median's lower middle value: against brute
  force over sorted (value, index) lists on tie-heavy integer data;
* the DG encoder (hicl_router.py:70-85): known answers — a 3-4-5 row normalises to 0.6/0.8,
  ties at the k-th place keep the lower indices, an all-negative row gives the zero vector;
* SoftMoE (gate.py:351-358): equal keys and values give 1/E; a sum below eps(bf16) = 0.078125
  divides by eps instead of the sum;
* Expert-Oriented (gate.py:361-366) with identity encoders: Σ_d silu(x_d) · silu(emb_e,d);
* with the auxiliary heads off: logits = (x·Wgᵀ + affinity[:, modal] + bias) / T, and the
  scores, top-k and weights follow by brute force;
* the temperature rules (gate.py:297-308) in bf16 and fp32, and the loss terms
  (gate.py:433-444, :556-610) on inputs whose means are known in closed form.
"""
import math

import numpy as np
import pytest
import torch

from oracle import moegate_oracle as mg


def _silu(v):
    return v / (1.0 + math.exp(-v))


def make_params(E=4, H=8, D=2, dg=16, M=3, seed=0, heads=None, **kw):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)
    p = mg.MoEGateParams(
        gate=r(E, H), dg_proj=r(dg, H), dg_bias=r(dg), prototypes=r(E, dg), got_proj=r(E, H),
        gate_k=r(E, H), gate_v=r(E, H), enc0=r(D, H), enc2=r(D, D), cap0=r(D, D), cap2=r(D, D),
        expert_embeddings=r(E, D), modal_affinity=r(E, M), expert_bias=r(E), w_hicl=0.0,
        w_got=0.0, w_soft=0.0, w_eo=0.0, temperature=1.0, temperature_max=5.0,
        usage_count=torch.zeros(E, dtype=torch.float64), total_routing_count=0.0)
    if heads is not None:
        p.heads = frozenset(heads)
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def test_topk_lower_index_brute_force():
    rng = np.random.default_rng(0)
    v = torch.from_numpy(rng.integers(0, 5, size=(40, 13)).astype(np.float64))
    vals, idx = mg.topk_lower_index(v, 6)
    for r in range(v.shape[0]):
        want = sorted(range(13), key=lambda i: (-float(v[r, i]), i))[:6]
        assert idx[r].tolist() == want
        assert vals[r].tolist() == [float(v[r, i]) for i in want]


@pytest.mark.parametrize("E", [1, 2, 7, 8, 64])
def test_lower_median_brute_force(E):
    rng = np.random.default_rng(E)
    v = torch.from_numpy(rng.integers(-3, 4, size=(25, E)).astype(np.float64))
    med = mg.lower_median(v)
    for r in range(v.shape[0]):
        assert float(med[r]) == sorted(v[r].tolist())[(E - 1) // 2]


def test_dg_sparse_known_answers():
    H, dg = 4, 8
    p = make_params(H=H, dg=dg)
    p.dg_proj = torch.zeros(dg, H, dtype=torch.float64)
    p.dg_proj[:H] = torch.eye(H, dtype=torch.float64)  # dg = [x, 0, 0, 0, 0] + bias
    p.dg_bias = torch.zeros(dg, dtype=torch.float64)
    p.sparsity_k = 2
    x = torch.tensor([[3.0, 4.0, 1.0, -2.0],      # keeps 3 and 4 -> 0.6, 0.8
                      [5.0, 5.0, 5.0, 1.0],       # tie at the 2nd place: indices 0 and 1
                      [-1.0, -2.0, -3.0, -4.0]],  # nothing positive: zero vector
                     dtype=torch.float64)
    s = mg.dg_sparse(x, p)
    want = torch.zeros(3, dg, dtype=torch.float64)
    want[0, 0], want[0, 1] = 0.6, 0.8
    want[1, 0] = want[1, 1] = 1.0 / math.sqrt(2.0)
    assert torch.allclose(s, want, atol=1e-15, rtol=0)
    # fewer positives than k: the positive ones, normalised
    p.sparsity_k = 3
    s = mg.dg_sparse(torch.tensor([[0.0, 2.0, -1.0, 0.0]], dtype=torch.float64), p)
    assert s[0, 1] == 1.0 and float(s.abs().sum()) == 1.0


def test_softmoe_known_answers():
    E, H = 4, 8
    p = make_params(E=E, H=H)
    p.gate_k = torch.zeros(E, H, dtype=torch.float64)
    p.gate_v = torch.zeros(E, H, dtype=torch.float64)
    x = torch.randn(3, H, dtype=torch.float64)
    soft = mg.head_logits(x, p)["soft"]
    assert torch.allclose(soft, torch.full((3, E), 1.0 / E, dtype=torch.float64), atol=1e-15)
    # keys [0, 1, 2] (median 1), values [10, -10, -10]: sigmoid ~ [0, 0.5, 1] times softmax
    # ~ [1, 2e-9, 2e-9] sums to ~3e-9 < eps, so the result is soft / eps, not soft / sum
    E = 3
    p = make_params(E=E, H=E, soft_temperature=0.01, eps=0.078125)
    p.gate_k = torch.diag(torch.tensor([0.0, 1.0, 2.0], dtype=torch.float64))
    p.gate_v = torch.diag(torch.tensor([10.0, -10.0, -10.0], dtype=torch.float64))
    x = torch.ones(1, E, dtype=torch.float64)
    soft = mg.head_logits(x, p)["soft"][0]
    lv = torch.tensor([10.0, -10.0, -10.0], dtype=torch.float64)
    sm = torch.exp(lv - 10.0) / torch.exp(lv - 10.0).sum()
    sw = torch.tensor([1 / (1 + math.exp(100.0)), 0.5, 1 / (1 + math.exp(-100.0))], dtype=torch.float64)
    assert float((sw * sm).sum()) < 0.078125
    assert torch.allclose(soft, sw * sm / 0.078125, rtol=1e-12, atol=0)


def test_expert_oriented_identity_encoders():
    E, H, D = 3, 5, 2
    p = make_params(E=E, H=H, D=D)
    p.enc0 = torch.zeros(D, H, dtype=torch.float64)
    p.enc0[0, 1] = p.enc0[1, 3] = 1.0             # picks x_1 and x_3
    for name in ("enc2", "cap0", "cap2"):
        setattr(p, name, torch.eye(D, dtype=torch.float64))
    x = torch.tensor([[0.1, -0.7, 2.0, 1.3, 9.0]], dtype=torch.float64)
    eo = mg.head_logits(x, p)["eo"][0]
    emb = p.expert_embeddings
    for e in range(E):
        # input side silu then identity; expert side identity, silu, identity
        want = _silu(-0.7) * _silu(float(emb[e, 0])) + _silu(1.3) * _silu(float(emb[e, 1]))
        assert abs(float(eo[e]) - want) < 1e-14


def test_heads_off_closed_form_and_routing():
    E, H, M, k = 6, 8, 3, 2
    p = make_params(E=E, H=H, M=M, seed=3, heads=(), temperature=2.5)
    x = torch.randn(2, 5, H, dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    modal = torch.tensor([2, 0])
    o = mg.moegate_forward(x, p, k, modal_id=modal)
    xf = x.reshape(-1, H)
    mids = [2] * 5 + [0] * 5
    for t in range(10):
        want = [(float(xf[t] @ p.gate[e]) + float(p.modal_affinity[e, mids[t]]) +
                 float(p.expert_bias[e])) / 2.5 for e in range(E)]
        assert np.allclose(o["logits"][t].numpy(), want, rtol=0, atol=1e-13)
        ex = [math.exp(v - max(want)) for v in want]
        sc = [v / sum(ex) for v in ex]
        top = sorted(range(E), key=lambda i: (-sc[i], i))[:k]
        assert o["indices"][t].tolist() == top
        wts = [math.exp(sc[i] - sc[top[0]]) for i in top]
        assert np.allclose(o["weights"][t].numpy(), [v / sum(wts) for v in wts], rtol=1e-12)
    # the budget term is absent without SoftMoE
    assert o["loss"] == pytest.approx(p.load_balance_alpha * float(
        ((o["scores"].mean(0) - 1.0 / E) ** 2).sum()) + p.z_loss_alpha * float((o["logits"] ** 2).mean()),
        rel=1e-12)


def test_effective_temperature_rules():
    bf = torch.bfloat16
    assert mg.effective_temperature(3.0, 5.0, 8191, bf) == 3.0
    # 3 * 0.3 = 0.9 rounds to the bf16 neighbour 0.8984375 (spacing 2^-8 in [0.5, 1))
    assert mg.effective_temperature(3.0, 5.0, 8192, bf) == 0.8984375
    assert mg.effective_temperature(3.0, 5.0, 8192, torch.float32) == float(np.float32(3.0) * np.float32(0.3))
    assert mg.effective_temperature(10.0, 5.0, 100, bf) == 5.0
    # the lower clamp is 0.1 in the buffers' dtype: bf16(0.1) = 0.10009765625
    assert mg.effective_temperature(0.2, 5.0, 9000, bf) == 0.10009765625
    assert mg.effective_temperature(0.05, 5.0, 10, torch.float32) == float(np.float32(0.1))


def test_loss_terms_closed_form():
    E, H = 4, 8
    bias = torch.tensor([1.0, 0.0, -1.0, 0.5], dtype=torch.float64)
    p = make_params(E=E, H=H, heads=("soft_moe",), expert_bias=bias, soft_budget=2.0,
                    usage_count=torch.tensor([30.0, 0.0, 5.0, 12.5], dtype=torch.float64),
                    total_routing_count=10.0)
    p.gate = torch.zeros(E, H, dtype=torch.float64)
    p.w_soft = 0.0          # SoftMoE computed (budget term) but weighted out of the logits
    p.modal_affinity = torch.zeros(E, 3, dtype=torch.float64)
    x = torch.randn(7, 1, H, dtype=torch.float64)
    o = mg.moegate_forward(x, p, 2)
    sc = torch.softmax(bias, 0)
    lb = 0.01 * float(((sc - 0.25) ** 2).sum())
    cap = 0.005 * ((3.0 - 1.2) ** 2 + (1.25 - 1.2) ** 2)    # usage 3.0 and 1.25 exceed 1.2
    z = 1e-4 * float((bias ** 2).mean())
    budget = 0.01 * (1.0 - 2.0) ** 2                           # each token's SoftMoE mass is 1
    assert o["loss"] == pytest.approx(lb + cap + z + budget, rel=1e-12)
