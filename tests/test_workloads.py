"""The skew recipe of cfg5 (pisceslx_amd/workloads.py), on the CPU.

cfg5 routes in fixed-shape mode with expert_bias_e = beta * ln(p_e), p_e ~ rank^-1.2 over a
seeded permutation, and 16 seeded experts held at -30 so they receive nothing. beta is the
value whose realised top-8 load is closest to the Zipf(1.2) target in KL; with top-8 routing
one expert can take at most one slot per token, so the heaviest Zipf shares (the first is
~0.26 of the slots, i.e. ~2.1 slots per token) are out of reach and the KL cannot reach 0.

The search is rerun here on cfg5's shape (8192 tokens, hidden 7168, 256 experts; x ~ N(0,1)
and the gate weight ~ N(0, 0.02) in bf16, drawn on the CPU generator — the GPU's draw differs in
its values, not in its statistics) and must return the beta the configuration uses.
"""
import numpy as np
import torch

from pisceslx_amd.workloads import SPECS, load_kl, zipf_beta_search, zipf_bias, zipf_target


def test_zipf_target_closed_form():
    p = zipf_target(256, 1.2, 16, 0)
    assert abs(p.sum() - 1.0) < 1e-12
    assert int((p == 0).sum()) == 16
    live = np.sort(p[p > 0])[::-1]
    ranks = np.arange(1, 241, dtype=np.float64)
    np.testing.assert_allclose(live / live[0], ranks ** -1.2, rtol=1e-12)
    # the bias puts the same tail experts at -30 and is beta * ln of the un-truncated shares
    b = zipf_bias(256, 1.2, 16, 0, beta=1.0)
    assert set(np.nonzero(b == -30.0)[0]) == set(np.nonzero(p == 0)[0])
    b2 = zipf_bias(256, 1.2, 16, 0, beta=2.0)
    live_b = b > -30.0
    np.testing.assert_allclose(b2[live_b], 2.0 * b[live_b], rtol=1e-6)


def test_load_kl_closed_forms():
    t = np.array([0.5, 0.25, 0.25, 0.0])
    assert load_kl([2, 1, 1, 0], t) == 0.0
    # all load on expert 0: KL = ln(1 / 0.5)
    assert abs(load_kl([7, 0, 0, 0], t) - np.log(2.0)) < 1e-15
    assert load_kl([1, 1, 1, 1], t) == float("inf")


def test_cfg5_beta_minimises_the_load_kl():
    spec = SPECS["cfg5"]
    g = torch.Generator().manual_seed(0)
    x = torch.randn(8192, spec.hidden, generator=g).to(torch.bfloat16).float()
    wg = (torch.randn(spec.num_experts, spec.hidden, generator=g) * 0.02).to(torch.bfloat16).float()
    logits = x @ wg.t()
    beta, kl = zipf_beta_search(logits, spec)
    print(f"cfg5 zipf beta {beta}, KL(realised || Zipf(1.2)) = {kl:.4f} nats", flush=True)
    assert beta == spec.zipf_beta
    assert 0.0 < kl < 0.2
    b = torch.from_numpy(zipf_bias(spec.num_experts, spec.zipf_s, spec.zero_experts, 0, beta))
    counts = np.bincount(torch.topk(logits + b, spec.top_k, dim=1).indices.reshape(-1).numpy(),
                         minlength=spec.num_experts)
    assert int((counts == 0).sum()) == spec.zero_experts
