"""The bf16 layer-output allowance (tests/helpers.py ``bf16_allowance``) pinned by the
reference's own arithmetic, on the CPU.

The GPU layer tests compare against the correctly rounded oracle (every GEMM of the layer
dtype summed exactly and rounded once). The reference runs the same chain with torch's bf16
``F.linear`` (``YvSwiGLUExpert.forward``, model/moe/expert.py:484-489; the shared experts'
fused gate/up, model/moe/layer.py:842-854), which sums in fp32 in torch's own order. This test
runs that chain (``layer_forward(..., reference_linear=True)``) on cfg4's 384-token batch — int4
g128 weights, 128 experts, top-8, one shared expert, the same logits and capacity — and
measures it against the correctly rounded oracle:

* elements above 2e-2 exist: 2e-2 alone does not hold between the reference and its own
  correctly rounded statement, so it cannot bind a third correct implementation either;
* every one of them lies at |out| >= 2, within two bf16 steps of the oracle (0.03125), and
  the whole output lies inside ``bf16_allowance``;
* at most 1e-5 of the elements exceed 2e-2 and the cosine is >= 0.9999 (the north star's
  other two figures).
"""
import numpy as np
import pytest
import torch

from pisceslx_amd.workloads import make_workload
from oracle import moe_oracle as mo

from helpers import BF16_MAX_ABS, bf16_allowance, bf16_ulp, cosine


def test_allowance_values():
    want = torch.tensor([0.5, 1.9, 2.0, 2.69, 3.99, 4.0, 5.0, 9.0], dtype=torch.bfloat16)
    got = bf16_allowance(want).tolist()
    assert got == [BF16_MAX_ABS, BF16_MAX_ABS, 0.03125, 0.03125, 0.03125, 0.03125, 0.03125, 0.0625]


@pytest.fixture(scope="module")
def cfg4_pair():
    w = make_workload("cfg4", device="cpu", n_tokens=384)
    p = mo.params_from_workload(w)
    lg = mo.router_logits(w.x, w.gate_weight)
    cap = mo.layer_capacity(p, w.x)
    exact = mo.layer_forward(w.x, p, logits=lg, cap=cap)["out"]
    ref = mo.layer_forward(w.x, p, logits=lg, cap=cap, reference_linear=True)["out"]
    return exact, ref


def test_reference_bf16_chain_envelope(cfg4_pair):
    exact, ref = cfg4_pair
    assert exact.dtype == torch.bfloat16 and ref.dtype == torch.bfloat16
    want, got = exact.double(), ref.double()
    d = (got - want).abs()
    over = d > BF16_MAX_ABS
    n_over = int(over.sum())
    print(f"reference bf16 chain vs correctly rounded (cfg4, N=384): max_abs={float(d.max()):.5f} "
          f"above 2e-2: {n_over}/{d.numel()} at |want| = {want[over].abs().tolist()}", flush=True)
    assert n_over >= 1
    assert bool((want[over].abs() >= 2.0).all())
    assert bool((d[over] <= 2 * bf16_ulp(exact)[over]).all())
    assert bool((d <= bf16_allowance(exact)).all())
    assert n_over <= 1e-5 * d.numel()
    assert cosine(got, want) >= 0.9999
    # the differences are whole bf16 steps: both chains end in a bf16 rounding
    steps = (d[over] / bf16_ulp(exact)[over]).numpy()
    assert np.all(steps == np.round(steps))
