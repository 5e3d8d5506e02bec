"""yvmoe_forward_static (the layer on the library's static scratch, no allocation) against
yvmoe_forward with a caller workspace: bit-identical outputs, shared outputs and routing, on
two calls in a row with the second one smaller, through the C ABI."""
import numpy as np
import pytest
import torch

from pisceslx_amd import _lib
from pisceslx_amd import functional as yvf
from pisceslx_amd.workloads import make_workload, mix_weights, router_state

pytestmark = pytest.mark.gpu


def _same_routing(a, b):
    for name in ("weights", "indices", "counts", "offsets", "perm", "pos", "capacity"):
        ta, tb = getattr(a, name), getattr(b, name)
        assert torch.equal(ta, tb), name


@pytest.mark.parametrize("name,sizes", [("cfg2", (64, 17)), ("cfg4", (40, 9))])
def test_static_scratch_matches_workspace_entry(cuda, name, sizes):
    w = make_workload(name, device=cuda, n_tokens=max(sizes))
    st, mix = router_state(w), mix_weights(w)
    H = w.spec.hidden
    g = torch.Generator(device=cuda).manual_seed(7)
    for n in sizes:
        print(f"static scratch {name} N={n}", flush=True)
        x = w.x[:n].contiguous()
        skip = torch.randn(n, H, device=cuda, generator=g).to(x.dtype)
        ref_out, ref_sh, ref_rt = yvf.moe_forward(x, st, w.experts, mix, skip)
        out, sh, rt = yvf.moe_forward_static(x, st, w.experts, mix, skip)
        torch.cuda.synchronize()
        assert torch.equal(out, ref_out)
        if w.spec.num_shared > 0:
            assert torch.equal(sh, ref_sh)
        _same_routing(rt, ref_rt)


def test_static_scratch_with_preallocated_outputs(cuda):
    """All outputs passed in: the whole call allocates nothing; a repeated call into the same
    buffers gives the same bits."""
    w = make_workload("cfg2", device=cuda, n_tokens=32)
    st, mix = router_state(w), mix_weights(w)
    N, H = w.x.shape
    out = torch.empty_like(w.x)
    sh = torch.empty_like(w.x)
    rt = yvf.Routing.empty(N, w.spec.num_experts, w.spec.top_k, cuda)
    ref = yvf.moe_forward(w.x, st, w.experts, mix, None)
    for _ in range(2):
        yvf.moe_forward_static(w.x, st, w.experts, mix, None, out=out, shared_out=sh, routing=rt)
        torch.cuda.synchronize()
        assert torch.equal(out, ref[0]) and torch.equal(sh, ref[1])
        _same_routing(rt, ref[2])


def test_static_scratch_rejects_oversized_batches(cuda):
    """A batch whose workspace exceeds the static scratch is rejected before any launch."""
    import ctypes
    w = make_workload("cfg2", device=cuda, n_tokens=8)
    st = router_state(w)
    n_big = 1024
    need = yvf.workspace_bytes(n_big, _lib.ACT_BF16, st, w.experts)
    assert need > _lib.STATIC_SCRATCH_BYTES
    r, e = st.struct(), w.experts.struct()
    rt = yvf.Routing.empty(8, w.spec.num_experts, w.spec.top_k, cuda)
    o = rt.struct()
    lib = _lib.lib()
    rc = lib.yvmoe_forward_static(w.x.data_ptr(), _lib.ACT_BF16, n_big, ctypes.byref(r),
                                  ctypes.byref(e), None, None, w.x.data_ptr(), None,
                                  ctypes.byref(o), torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.YVMOE_ERR_WORKSPACE
    assert b"static" in lib.yvmoe_last_error()
    np.testing.assert_equal(int(rc), _lib.YVMOE_ERR_WORKSPACE)
