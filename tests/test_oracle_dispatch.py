"""Pins the oracle's dispatch (oracle/moe_oracle.py: dispatch_forward, the CPU statement of
PiscesLxFusedMoEDispatch.forward, opss/infer/fused_moe.py:54-123) independently of its own
sort / gather / scatter:

* against a sort-free statement: every (token, slot) run through its expert on its own, the
  slots of a token summed in slot order — the same arithmetic with no permutation, so a wrong
  argsort, a wrong inverse permutation or a token/slot mix-up changes bits;
* counts / offsets / the expert-sorted order against their definitions on hand-built indices
  (duplicates inside a token, empty experts, indices outside [0, E));
* against the layer oracle: dispatching the layer oracle's own routing reproduces its routed
  output bit for bit (a layer with no shared experts);
* a one-hot construction whose combine has a closed form.
"""
import numpy as np
import torch

from oracle import moe_oracle as mo


def _experts(E, H, F, seed):
    g = torch.Generator().manual_seed(seed)
    ws = [tuple((torch.randn(o, i, generator=g) * 0.2).to(torch.bfloat16).float()
                for o, i in ((F, H), (F, H), (H, F))) for _ in range(E)]
    return lambda e: ws[e]


def _sort_free(x, w, idx, E, fn):
    N, k = idx.shape
    out = torch.zeros(N, x.shape[1], dtype=torch.float32)
    for t in range(N):
        acc = torch.zeros(x.shape[1], dtype=torch.float32)
        for j in range(k):
            e = int(idx[t, j])
            if not 0 <= e < E:
                continue
            wg, wu, wd = fn(e)
            y = mo.swiglu(x[t:t + 1], wg.to(x.dtype), wu.to(x.dtype), wd.to(x.dtype)).float()[0]
            acc = acc + torch.tensor(w[t, j], dtype=torch.float32) * y
        out[t] = acc
    return out.to(x.dtype)


def test_dispatch_matches_sort_free_statement():
    E, H, F, N, k = 5, 64, 96, 13, 3
    fn = _experts(E, H, F, 0)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(N, H, generator=g).to(torch.bfloat16)
    rng = np.random.default_rng(2)
    idx = rng.integers(0, E, size=(N, k))
    idx[3] = [1, 1, 1]          # the same expert three times in one token
    idx[4, 2] = E               # an index past the last expert
    idx[5, 0] = -1              # a negative one
    idx[idx == 4] = 0           # expert 4 receives nothing
    w = rng.random((N, k)).astype(np.float32)
    w[6] = 0.0                  # zero-weight slots are computed and add zero
    d = mo.dispatch_forward(x, w, idx, E, fn)
    ref = _sort_free(x, w, idx, E, fn)
    assert torch.equal(d.out, ref)
    assert d.invalid == 2
    assert torch.equal(d.out[6], torch.zeros(H, dtype=torch.bfloat16))


def test_counts_offsets_and_order_by_definition():
    E, N, k = 6, 7, 2
    idx = np.array([[3, 0], [3, 3], [5, 0], [0, 7], [2, 3], [-2, 2], [0, 0]])
    d = mo.dispatch_forward(torch.zeros(N, 64, dtype=torch.bfloat16), np.ones((N, k)), idx, E,
                            _experts(E, 64, 64, 3))
    assert d.counts.tolist() == [5, 0, 2, 4, 0, 1]
    assert d.offsets.tolist() == [0, 5, 5, 7, 11, 11, 12]
    assert d.invalid == 2
    # expert-sorted order of the flat slots t * k + j, ties in slot order: expert 0 holds
    # slots 1, 5, 6, 12, 13; expert 2 slots 8, 11; expert 3 slots 0, 2, 3, 9; expert 5 slot 4;
    # slots 7 and 10 (indices 7 and -2) have no place
    assert d.perm.tolist() == [1, 5, 6, 12, 13, 8, 11, 0, 2, 3, 9, 4]


def test_dispatch_of_layer_routing_equals_layer_routed_output():
    from pisceslx_amd.workloads import make_workload
    w = make_workload("cfg5", device="cpu", n_tokens=40, num_experts=16, hidden=256, ffn=256)
    params = mo.params_from_workload(w)
    assert params.num_shared == 0
    lay = mo.layer_forward(w.x, params)
    r = lay["routing"]
    d = mo.dispatch_forward(w.x, r.weights, r.indices, params.num_experts, params.expert)
    assert torch.equal(d.out, lay["out"])
    assert np.array_equal(d.counts, r.counts) and np.array_equal(d.perm, r.perm)


def test_one_hot_combine_closed_form():
    # expert e maps x to c_e * e_0 exactly (one-hot gate/up rows, a scaled down column), so
    # out[t] = sum_j w[t,j] * y_e exactly in fp32
    E, H, F, N, k = 3, 64, 64, 4, 2
    ws = []
    for e in range(E):
        wg = torch.zeros(F, H)
        wu = torch.zeros(F, H)
        wd = torch.zeros(H, F)
        wg[0, 0] = 4.0          # gate = 4 x_0
        wu[0, 0] = 1.0          # up = x_0
        wd[0, 0] = float(e + 1)  # y_0 = (e + 1) * silu(4 x_0) * x_0
        ws.append((wg, wu, wd))
    x = torch.zeros(N, H, dtype=torch.float32)
    x[:, 0] = 1.0
    idx = np.array([[0, 1], [2, 2], [1, 0], [2, 0]])
    w = np.array([[0.25, 0.75], [0.5, 0.5], [1.0, 0.0], [0.125, 0.875]], dtype=np.float32)
    d = mo.dispatch_forward(x, w, idx, E, lambda e: ws[e])
    s = torch.tensor(4.0) * torch.sigmoid(torch.tensor(4.0))  # silu(4)
    s = float(s)
    for t in range(N):
        want = 0.0
        for j in range(k):
            want = np.float32(want + np.float32(w[t, j]) * np.float32((idx[t, j] + 1) * s))
        assert abs(float(d.out[t, 0]) - float(want)) <= 2e-6 * abs(float(want))
        assert torch.count_nonzero(d.out[t, 1:]) == 0
