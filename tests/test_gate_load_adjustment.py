"""YvStableMoEGate's load adjustment (model/moe/gate.py:1192-1209, _predict_future_load
:1030-1057) — the host-side bias vector the routing kernels add to the logits — pinned by
closed forms on constructed gate states (CPU, no GPU):

* no history (history_ptr == 0): no adjustment;
* fewer than 10 load records: the uniform prediction 1/E, so the adjustment is
  0.1 * (1/E - mean(routing_history[:history_ptr]));
* 10 or more records: the LSTM prediction. With every LSTM weight zero the recurrence no
  longer reads its input: each layer's cell follows c_t = f c_{t-1} + i g from its biases
  alone, c_T = i g (1 - f^T) / (1 - f), h_T = o tanh(c_T), so the prediction head sees a
  known constant vector and the prediction is softmax over experts of the mean over the
  horizon of (h_T * rowsum(W_head) + b_head) viewed [E, horizon] — a transposed view, a mean
  over the wrong axis or a record count off by one changes it;
* a usage history whose entropy is below 0.7 of log(E) (the reference adds random noise
  there, gate.py:1206-1209) raises NotImplementedError;
* the adjustment is cached on the buffers' versions and recomputed when they change.
"""
import math

import numpy as np
import pytest
import torch

from pisceslx_amd.gate import YvStableMoEGate

E, H, HORIZON = 8, 64, 10


def _gate():
    torch.manual_seed(0)
    return YvStableMoEGate(H, E, top_k=2, device="cpu").eval()


def _usage_rows(n, seed):
    """n usage rows (each a distribution over experts) whose mean has high entropy."""
    rng = np.random.default_rng(seed)
    rows = rng.dirichlet(np.full(E, 20.0), size=n)
    return rows


def _set_history(g, rows, load_rows=None):
    with torch.no_grad():
        g.routing_history[:len(rows)] = torch.tensor(rows, dtype=torch.float32)
        g.history_ptr.fill_(len(rows))
        if load_rows is not None:
            g.expert_load_buffer[:len(load_rows)] = torch.tensor(load_rows, dtype=torch.float32)
            g.load_buffer_ptr.fill_(len(load_rows))


def test_no_history_no_adjustment():
    g = _gate()
    assert g._load_adjustment() is None


def test_uniform_prediction_below_ten_records():
    g = _gate()
    rows = _usage_rows(5, 1)
    _set_history(g, rows, load_rows=_usage_rows(9, 2))   # 9 < 10 load records
    adj = g._load_adjustment()
    recent = rows.astype(np.float32).astype(np.float64).mean(axis=0)
    want = 0.1 * (1.0 / E - recent)
    np.testing.assert_allclose(adj.numpy(), want, rtol=0, atol=1e-7)


def _lstm_closed_form(biases, T):
    """h_T of a 2-layer LSTM with zero weights: per layer (b_i, b_f, b_g, b_o) biases."""
    sig = lambda v: 1.0 / (1.0 + math.exp(-v))
    h = None
    for bi, bf, bg, bo in biases:
        i, f, gg, o = sig(bi), sig(bf), math.tanh(bg), sig(bo)
        c = i * gg * (1.0 - f ** T) / (1.0 - f)
        h = o * math.tanh(c)
    return h


@pytest.mark.parametrize("T", [10, 12, 37])
def test_lstm_prediction_closed_form(T):
    g = _gate()
    biases = [(0.5, 1.0, 0.8, -0.3), (-0.2, 0.3, 1.5, 0.7)]
    lstm = g.load_predictor
    rng = np.random.default_rng(3)
    W = rng.normal(0, 0.5, size=(E * HORIZON, 64))
    b = rng.normal(0, 0.5, size=E * HORIZON)
    with torch.no_grad():
        for name, p in lstm.named_parameters():
            p.zero_()
        for layer, (bi, bf, bg, bo) in enumerate(biases):
            getattr(lstm, f"bias_ih_l{layer}").copy_(torch.tensor(
                [bi] * 64 + [bf] * 64 + [bg] * 64 + [bo] * 64))
        g.predictor_head.weight.copy_(torch.tensor(W, dtype=torch.float32))
        g.predictor_head.bias.copy_(torch.tensor(b, dtype=torch.float32))
    rows = _usage_rows(7, 4)
    _set_history(g, rows, load_rows=_usage_rows(T, 5))
    adj = g._load_adjustment()
    hT = _lstm_closed_form(biases, T)
    Wf = W.astype(np.float32).astype(np.float64)
    bf_ = b.astype(np.float32).astype(np.float64)
    pred = (hT * Wf.sum(axis=1) + bf_).reshape(E, HORIZON).mean(axis=1)
    predicted = np.exp(pred - pred.max())
    predicted /= predicted.sum()
    recent = rows.astype(np.float32).astype(np.float64).mean(axis=0)
    want = 0.1 * (predicted - recent)
    np.testing.assert_allclose(adj.numpy(), want, rtol=0, atol=2e-6)
    # the prediction is not uniform: the LSTM path was taken
    assert np.abs(predicted - 1.0 / E).max() > 1e-2


def test_unbalanced_history_raises():
    g = _gate()
    rows = np.zeros((4, E))
    rows[:, 0] = 1.0          # all traffic on one expert: entropy 0 < 0.7 log(E)
    _set_history(g, rows)
    with pytest.raises(NotImplementedError, match="balance_ratio"):
        g._load_adjustment()


def test_balance_ratio_threshold():
    """The noise condition balance_ratio = H(recent) / log(E) < 0.7 (gate.py:1198-1206): a
    mixture of one-hot and uniform rows placed just above and just below the threshold."""
    def mix_for(ratio_target):
        # recent = a * onehot + (1 - a) * uniform; find a with entropy ratio = target
        lo, hi = 0.0, 1.0
        for _ in range(60):
            a = 0.5 * (lo + hi)
            p = np.full(E, (1 - a) / E)
            p[0] += a
            r = -(p * np.log(p)).sum() / math.log(E)
            lo, hi = (a, hi) if r > ratio_target else (lo, a)
        return a

    for target, raises in ((0.72, False), (0.68, True)):
        a = mix_for(target)
        g = _gate()
        row = np.full(E, (1 - a) / E)
        row[0] += a
        _set_history(g, np.stack([row, row]))
        if raises:
            with pytest.raises(NotImplementedError):
                g._load_adjustment()
        else:
            adj = g._load_adjustment()
            np.testing.assert_allclose(adj.numpy(), 0.1 * (1.0 / E - row.astype(np.float32)),
                                       rtol=0, atol=1e-7)


def test_adjustment_cache_follows_buffer_versions():
    g = _gate()
    rows = _usage_rows(3, 6)
    _set_history(g, rows)
    a1 = g._load_adjustment()
    assert g._load_adjustment() is a1          # cached: no recomputation, no device sync
    rows2 = _usage_rows(3, 7)
    _set_history(g, rows2)                     # in-place writes bump the buffers' versions
    a2 = g._load_adjustment()
    want = 0.1 * (1.0 / E - rows2.astype(np.float32).astype(np.float64).mean(axis=0))
    np.testing.assert_allclose(a2.numpy(), want, rtol=0, atol=1e-7)
