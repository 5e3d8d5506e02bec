"""YvMoEGate on the GPU against the CPU oracle (oracle/moegate_oracle.py).

For each case the module's fp32 logits (yvmoe_moegate_logits) are compared with the oracle's
float64 logits (max-abs <= 1e-4 · max(1, max |logit|)), the routing is checked bit for bit
against the C routing oracle given the GPU's logits (indices, weights, counts, permutation),
``top_scores`` are those weights in x's dtype, and the loss is within 1e-4 relative of the
oracle's. Cases: the decode shape of the 7B-style layer (hidden 4096, 64 experts, top-6,
64 tokens), a prefill sample, heads weighted up so every head moves the logits by O(1), exact
ties at the 32nd DG activation, more candidates than the ranking takes (exact radix
select), fewer than 32 positive DG activations, modal ids, a pruned
head, the long-sequence temperature, fp32 activations, N = 0, determinism, and the PathMoE
stage cache; and the bench's 16,721-token prefill shape at full size on sampled tokens.
"""
import numpy as np
import pytest
import torch

from oracle import moegate_oracle as mg
from pisceslx_amd.gate import YvMoEGate

pytestmark = pytest.mark.gpu


def _gate(H, E, k, dtype=torch.bfloat16, seed=0, scale_heads=False, stage=1):
    torch.manual_seed(seed)
    g = YvMoEGate(H, E, top_k=k, dtype=dtype)
    with torch.no_grad():
        g.expert_modal_affinity.normal_(0.0, 0.3)
        g.expert_bias.normal_(0.0, 0.2)
        g.hicl_dg_encoder.dg_bias.normal_(0.0, 0.05)
        if scale_heads:
            for name in ("w_hicl", "w_got", "w_soft", "w_expert_orient"):
                getattr(g, name).fill_(1.0)
            g.hicl_prototypes.mul_(50.0)
    g._path_moe_stage_size = stage
    return g.cuda().eval()


def _check(g, x, oracle, modal_id=None, heads=None):
    B, S, H = x.shape
    E, k = g.num_experts, min(g.top_k, g.num_experts)
    print(f"moegate B={B} S={S} H={H} E={E} k={k} dtype={x.dtype}", flush=True)
    scores, idx, loss = g(x, modal_id=modal_id)
    torch.cuda.synchronize()
    lg = g.last_logits.cpu().numpy()
    p = mg.params_from_state_dict(g.state_dict(), g.gate.weight.dtype,
                                  soft_temperature=g.soft_moe_temperature, heads=heads)
    o = mg.moegate_forward(x.cpu(), p, k, modal_id=None if modal_id is None else modal_id.cpu())
    ref = o["logits"].numpy()
    tol = 1e-4 * max(1.0, float(np.abs(ref).max())) if ref.size else 1e-4
    err = float(np.abs(lg - ref).max()) if ref.size else 0.0
    print(f"  logits max_abs={err:.3e} (tol {tol:.1e})", flush=True)
    assert err <= tol
    r = oracle.route(lg.astype(np.float32), k, -1, None)
    routing = g.last_routing
    assert np.array_equal(idx.cpu().numpy(), r.indices.astype(np.int64))
    assert np.array_equal(routing.weights.cpu().numpy().view(np.uint32), r.weights.view(np.uint32))
    assert np.array_equal(routing.counts.cpu().numpy(), r.counts)
    assert np.array_equal(routing.perm.cpu().numpy(), r.perm)
    assert scores.dtype == x.dtype and torch.equal(scores, routing.weights.to(x.dtype))
    got_loss, want_loss = float(loss), o["loss"]
    print(f"  loss {got_loss:.6e} oracle {want_loss:.6e}", flush=True)
    if x.dtype == torch.bfloat16:
        assert got_loss == pytest.approx(float(torch.tensor(want_loss).to(torch.bfloat16)), rel=1e-2)
    assert float(g._last_loss_f32) == pytest.approx(want_loss, rel=1e-4, abs=1e-7)
    return o


@pytest.mark.parametrize("B,S,H,E,k,scale", [
    (64, 1, 4096, 64, 6, False),   # 7B-style decode: 64 sequences x 1 token
    (64, 1, 4096, 64, 6, True),    # every head weighted 1
    (2, 200, 1024, 8, 2, True),    # small layer, prefill-like
    (3, 37, 5120, 128, 8, False),  # hidden 5120: DG width 20480
    (1, 40, 7168, 256, 8, True),   # hidden 7168, 256 experts: DG width 28672
])
def test_moegate_matches_oracle(cuda, oracle, B, S, H, E, k, scale):
    g = _gate(H, E, k, scale_heads=scale, seed=H + E)
    x = torch.randn(B, S, H, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).cuda()
    _check(g, x, oracle)


def test_dg_ties_and_few_positives(cuda, oracle):
    H, E = 256, 8
    g = _gate(H, E, 2, scale_heads=True, seed=1)
    dg = g.hicl_dg_encoder
    with torch.no_grad():
        dg.dg_proj.weight.zero_()           # DG activations = relu(dg_bias) for every token
        b = torch.full((dg.dg_dim,), -1.0)
        b[torch.arange(3, 93, 3)] = 2.0     # 30 entries above the threshold
        b[[700, 5, 1000, 11, 400]] = 1.0     # five-way tie for the last two places
        dg.dg_bias.copy_(b)
    x = torch.randn(2, 9, H, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).cuda()
    _check(g, x, oracle)
    with torch.no_grad():                   # 10 positive activations only
        b = torch.full((dg.dg_dim,), -1.0)
        b[torch.arange(0, 1000, 100)] = torch.linspace(0.5, 1.5, 10)
        dg.dg_bias.copy_(b)
    _check(g, x, oracle)
    with torch.no_grad():                   # none positive: HiCL adds 0
        dg.dg_bias.fill_(-1.0)
    _check(g, x, oracle)


def test_dg_exact_select_beyond_candidates(cuda, oracle):
    H, E = 1024, 8                          # DG width 4096
    g = _gate(H, E, 2, scale_heads=True, seed=3)
    dg = g.hicl_dg_encoder
    x = torch.randn(2, 5, H, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16).cuda()
    with torch.no_grad():                   # ~1500 candidates tie at the bound: exact select
        dg.dg_proj.weight.zero_()
        b = torch.full((dg.dg_dim,), -1.0)
        b[torch.arange(1, 1001, 2)] = 1.0
        b[torch.arange(2, 3002, 3)] = 1.0
        b[[17, 900, 40, 3]] = torch.tensor([2.0, 3.0, 2.5, 2.0])
        dg.dg_bias.copy_(b)
    _check(g, x, oracle)
    with torch.no_grad():                   # every activation equal
        dg.dg_bias.fill_(0.5)
    _check(g, x, oracle)
    with torch.no_grad():                   # 2000 distinct values above the bound
        b = torch.full((dg.dg_dim,), -1.0)
        b[1000:3000] = 1.0 + torch.arange(2000) * 1e-3
        dg.dg_bias.copy_(b)
    _check(g, x, oracle)


def test_modal_ids_and_pruned_head(cuda, oracle):
    H, E = 512, 16
    g = _gate(H, E, 4, scale_heads=True, seed=4)
    x = torch.randn(4, 16, H, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).cuda()
    _check(g, x, oracle, modal_id=torch.tensor([0, 6, 3, 1]))                    # per sequence
    _check(g, x, oracle, modal_id=torch.randint(0, 7, (4, 16), generator=torch.Generator().manual_seed(0)))
    with pytest.raises(IndexError):
        g(x, modal_id=torch.tensor([0, 7, 3, 1]))
    with torch.no_grad():
        g.sparse_gate_got.fill_(-10.0)
    g.prune_routing_heads(0.05)
    assert g._pruned_heads == {"got"} and not hasattr(g, "w_got")
    _check(g, x, oracle, heads=("hicl", "soft_moe", "expert_orient"))


def test_long_sequence_temperature_and_fp32(cuda, oracle):
    H, E = 256, 8
    g = _gate(H, E, 2, seed=6)
    x = torch.randn(1, 8192, H, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).cuda()
    o = _check(g, x, oracle)
    assert o["temperature"] == 0.8984375    # bf16(3.0 * 0.3)
    g32 = _gate(H, E, 2, dtype=torch.float32, seed=7, scale_heads=True)
    x32 = torch.randn(3, 50, H, generator=torch.Generator().manual_seed(8)).cuda()
    _check(g32, x32, oracle)


def test_empty_batch_and_determinism(cuda, oracle):
    H, E = 1024, 8
    g = _gate(H, E, 2, seed=9)
    s, i, loss = g(torch.zeros(1, 0, H, dtype=torch.bfloat16, device="cuda"))
    torch.cuda.synchronize()
    assert s.shape == (0, 2) and i.shape == (0, 2) and torch.isnan(loss)
    x = torch.randn(8, 300, H, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).cuda()
    g(x)
    a = g.last_logits.clone()
    la = g._last_loss_f32.clone()
    g(x)
    assert torch.equal(a, g.last_logits) and torch.equal(la, g._last_loss_f32)


def test_path_moe_stage_cache(cuda):
    H, E = 256, 8
    g = _gate(H, E, 2, seed=2, stage=4)
    gen = torch.Generator().manual_seed(0)
    xs = [torch.randn(2, 5, H, generator=gen).to(torch.bfloat16).cuda() for _ in range(6)]
    outs = [g(x)[1].clone() for x in xs[:5]]
    fresh = [g.last_routing]
    # calls 2-4 of a stage reuse call 1's routing; call 5 starts a new stage
    for j in (1, 2, 3):
        assert torch.equal(outs[j], outs[0])
    g2 = _gate(H, E, 2, seed=2, stage=1)
    assert torch.equal(outs[4], g2(xs[4])[1])
    # another token count resets the stage
    y = torch.randn(1, 7, H, generator=gen).to(torch.bfloat16).cuda()
    assert torch.equal(g(y)[1], g2(y)[1])
    assert fresh[0] is not None


# Batches of 1024 tokens and more take the wavefront-per-token form (a gate of at most 64
# experts): the same checks, and the DG selection cases that reach its buffer compaction
# (entries tied at the threshold, more candidates than the buffer holds, few positives).
@pytest.mark.parametrize("B,S,H,E,k,scale", [
    (4, 300, 1024, 64, 6, False),
    (2, 520, 2048, 32, 4, True),
    # hidden 4096, 64 experts: a 16,896-column projection over 5 row tiles of 256 (the last
    # holding 16 rows), 330 tiles, so the projection takes the wide four-wavefront form
    (1, 1040, 4096, 64, 6, False),
])
def test_moegate_wave_form_matches_oracle(cuda, oracle, B, S, H, E, k, scale):
    g = _gate(H, E, k, scale_heads=scale, seed=H + E + 1)
    x = torch.randn(B, S, H, generator=torch.Generator().manual_seed(7)).to(torch.bfloat16).cuda()
    _check(g, x, oracle)


def test_moegate_wave_form_dg_selection_cases(cuda, oracle):
    H, E = 1024, 16                          # DG width 4096
    g = _gate(H, E, 2, scale_heads=True, seed=9)
    dg = g.hicl_dg_encoder
    x = torch.randn(2, 530, H, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16).cuda()
    with torch.no_grad():                    # ~1500 entries tie at the 32nd place
        dg.dg_proj.weight.zero_()
        b = torch.full((dg.dg_dim,), -1.0)
        b[torch.arange(1, 1001, 2)] = 1.0
        b[torch.arange(2, 3002, 3)] = 1.0
        b[[17, 900, 40, 3]] = torch.tensor([2.0, 3.0, 2.5, 2.0])
        dg.dg_bias.copy_(b)
    _check(g, x, oracle)
    with torch.no_grad():                    # every activation equal: the 32 lowest indices
        dg.dg_bias.fill_(0.5)
    _check(g, x, oracle)
    with torch.no_grad():                    # values rising with the index: every entry enters
        dg.dg_bias.copy_(torch.linspace(0.01, 2.0, dg.dg_dim))
    _check(g, x, oracle)
    with torch.no_grad():                    # values falling with the index: the first 32 stay
        dg.dg_bias.copy_(torch.linspace(2.0, 0.01, dg.dg_dim))
    _check(g, x, oracle)
    with torch.no_grad():                    # 10 positive activations only
        b = torch.full((dg.dg_dim,), -1.0)
        b[torch.arange(0, 1000, 100)] = torch.linspace(0.5, 1.5, 10)
        dg.dg_bias.copy_(b)
    _check(g, x, oracle)
    with torch.no_grad():                    # random weights, a five-way tie at the last places
        dg.dg_proj.weight.normal_(0.0, 0.02)
        b = torch.full((dg.dg_dim,), -3.0)
        b[torch.arange(3, 93, 3)] = 4.0
        b[[700, 5, 1000, 11, 400]] = 3.5
        dg.dg_bias.copy_(b)
    _check(g, x, oracle)


def test_moegate_full_size_prefill_sampled_tokens(cuda, oracle):
    """The bench's prefill gate shape at full size: one sequence of 16,721 tokens, hidden 4096,
    64 experts, top-6, every head weighted 1 (the wide projection over 66 row tiles, the
    wavefront-per-token selection over 1,024 work-groups, the loss over their sums, the long-
    sequence temperature). Checked: the logits of 64 sampled tokens against the float64 oracle
    (temperature rule at the full sequence length), the routing of every token bit for bit
    against the C oracle given the GPU's logits, and the loss against the oracle's loss formula
    over every token's GPU logits and float64 SoftMoE weights."""
    from oracle import moegate_oracle as mgo
    H, E, k, N = 4096, 64, 6, 16721
    g = _gate(H, E, k, scale_heads=True, seed=11)
    x = torch.randn(1, N, H, generator=torch.Generator().manual_seed(12)).to(torch.bfloat16)
    print(f"moegate full size N={N} H={H} E={E} k={k}", flush=True)
    scores, idx, loss = g(x.cuda())
    torch.cuda.synchronize()
    lg = g.last_logits.cpu()
    p = mgo.params_from_state_dict(g.state_dict(), g.gate.weight.dtype,
                                   soft_temperature=g.soft_moe_temperature)
    tokens = np.sort(np.random.default_rng(13).choice(N, 64, replace=False))
    o = mgo.moegate_forward(x[0, tokens][None], p, k, seq_len=N)
    assert o["temperature"] == 0.8984375  # bf16(3.0 * 0.3): the long-sequence rule applied
    ref = o["logits"].numpy()
    got = lg[tokens].numpy()
    tol = 1e-4 * max(1.0, float(np.abs(ref).max()))
    err = float(np.abs(got - ref).max())
    print(f"  sampled logits max_abs={err:.3e} (tol {tol:.1e})", flush=True)
    assert err <= tol
    r = oracle.route(lg.numpy().astype(np.float32), k, -1, None)
    routing = g.last_routing
    assert np.array_equal(idx.cpu().numpy(), r.indices.astype(np.int64))
    assert np.array_equal(routing.weights.cpu().numpy().view(np.uint32), r.weights.view(np.uint32))
    assert np.array_equal(routing.counts.cpu().numpy(), r.counts)
    assert np.array_equal(routing.perm.cpu().numpy(), r.perm)
    want_loss = mgo.gate_loss(lg.double(), mgo.soft_weights(x[0].double(), p), p)
    print(f"  loss {float(g._last_loss_f32):.6e} oracle formula {want_loss:.6e}", flush=True)
    assert float(g._last_loss_f32) == pytest.approx(want_loss, rel=1e-4, abs=1e-7)
