"""The router GEMM (yvmoe_router_logits) on the GPU against float64, across the shapes its
forms take: the streaming form with 16 K splits up to 256 tokens; above, the LDS-tiled form with
K splits chosen per shape, including a partial last column block (router operand widths
Ep + 192 that are not multiples of 256) and splits whose last one is shorter.

Every logit within 2e-4 * max(1, max |logit|) of x @ gate.weight^T computed in float64 from the
same bf16 operands; the call is deterministic (two calls give the same bits).
"""
import ctypes

import numpy as np
import pytest
import torch

from pisceslx_amd import _lib
from pisceslx_amd import functional as yvf
from pisceslx_amd.functional import RouterState
from pisceslx_amd.quant import pack_router

pytestmark = pytest.mark.gpu


def _router(E, H, dev, seed):
    g = torch.Generator().manual_seed(seed)
    gw = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16)
    w1 = torch.randn(_lib.PREDICTOR_DIM, H, generator=g) * 0.02
    st = RouterState(E, H, min(6, E), False, True, 4, 1.0,
                     pack_router(gw.to(dev), w1.to(dev), _lib.ACT_BF16), None, None, None, None)
    return gw, st


@pytest.mark.parametrize("N,H,E", [
    (64, 4096, 64),     # decode: streaming form, 16 K splits
    (257, 1024, 8),     # just above the small-batch bound; ld 208: one partial column block
    (300, 4096, 64),    # ld 256: whole column block, 16 splits
    (777, 3072, 40),    # ld 240
    (1000, 2048, 128),  # ld 320: a whole and a partial column block
    (2000, 7168, 256),  # ld 448
    (4344, 5120, 128),  # cfg4's shape: 7 splits of 12 k-steps, the last of 8
    (600, 2048, 80),    # ld 272: the last column block holds one 16-column block
    (513, 64, 16),      # K = 64: one k-step, no split
])
def test_router_logits_against_float64(cuda, N, H, E):
    gw, st = _router(E, H, cuda, seed=N + H + E)
    x = (torch.randn(N, H, generator=torch.Generator().manual_seed(N)) * 1.0).to(torch.bfloat16)
    splits = _lib.lib().yvmoe_router_workspace_bytes(N, _lib.ACT_BF16, ctypes.byref(st.struct()))
    print(f"router N={N} H={H} E={E} partial-sum workspace {splits} B", flush=True)
    xd = x.to(cuda)
    lg = yvf.router_logits(xd, st)
    lg2 = yvf.router_logits(xd, st)
    torch.cuda.synchronize()
    assert torch.equal(lg, lg2)
    got = lg[:, :E].cpu().numpy()
    want = (x.double() @ gw.double().t()).numpy()
    tol = 2e-4 * max(1.0, float(np.abs(want).max()))
    err = float(np.abs(got - want).max())
    print(f"  max |err| {err:.3e} (bound {tol:.3e})", flush=True)
    assert err <= tol
