"""The layer forward captured in a HIP graph (torch.cuda.CUDAGraph) and replayed: the entry
points synchronize nothing with the host and allocate nothing (workspace and outputs from the
caller, or the library's static scratch), so the whole step — router GEMM, routing, expert
FFN, combine — records as kernels only. Every replay, with new inputs copied into the captured
buffers and eager work and host synchronizations between replays, must equal the eager call
on the same inputs bit for bit."""
import pytest
import torch

from pisceslx_amd import _lib
from pisceslx_amd import functional as yvf
from pisceslx_amd.workloads import make_workload, mix_weights, router_state

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,n,static", [("cfg2", 64, False), ("cfg2", 64, True),
                                           ("cfg3", 1024, False), ("cfg5", 256, True)])
def test_layer_graph_replays_match_eager(cuda, name, n, static):
    kw = {"num_experts": 32} if name == "cfg5" else {}
    w = make_workload(name, device=cuda, n_tokens=n, **kw)
    st, mix = router_state(w), mix_weights(w)
    N, H = w.x.shape
    E, k, S = w.spec.num_experts, w.spec.top_k, w.spec.num_shared
    x = w.x.clone()
    skip = torch.zeros_like(x)
    out = torch.empty_like(x)
    sh = torch.empty_like(x) if S > 0 else None
    rt = yvf.Routing.empty(N, E, k, cuda)
    ws = torch.empty(yvf.workspace_bytes(N, _lib.ACT_BF16, st, w.experts), dtype=torch.uint8,
                     device=cuda)

    def step():
        if static:
            yvf.moe_forward_static(x, st, w.experts, mix, skip if S > 0 else None, out=out,
                                   shared_out=sh, routing=rt)
        else:
            o = rt.struct()
            r, e = st.struct(), w.experts.struct()
            import ctypes
            _lib.check(_lib.lib().yvmoe_forward(
                x.data_ptr(), _lib.ACT_BF16, N, ctypes.byref(r), ctypes.byref(e),
                None if mix is None else mix.data_ptr(), skip.data_ptr() if S > 0 else None,
                out.data_ptr(), None if sh is None else sh.data_ptr(), ctypes.byref(o),
                ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream), "yvmoe_forward")

    side = torch.cuda.Stream(cuda)
    side.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(side):
        step()                                   # warm the launch path outside the capture
    torch.cuda.current_stream(cuda).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    gen = torch.Generator(device=cuda).manual_seed(9)
    for rep in range(4):
        print(f"graph {name} N={n} static={static} replay {rep}", flush=True)
        x.copy_(torch.randn(N, H, device=cuda, generator=gen).to(x.dtype))
        skip.copy_(torch.randn(N, H, device=cuda, generator=gen).to(x.dtype))
        graph.replay()
        torch.cuda.synchronize()
        g_out = out.clone()
        g_sh = None if sh is None else sh.clone()
        g_idx, g_w, g_perm = rt.indices.clone(), rt.weights.clone(), rt.perm.clone()
        # eager on the same inputs (other allocations and launches in between)
        e_out, e_sh, e_rt = yvf.moe_forward(x, st, w.experts, mix, skip if S > 0 else None)
        torch.cuda.synchronize()
        assert torch.equal(g_out, e_out), f"replay {rep}: output"
        if sh is not None:
            assert torch.equal(g_sh, e_sh), f"replay {rep}: shared output"
        assert torch.equal(g_idx, e_rt.indices) and torch.equal(g_w, e_rt.weights)
        assert torch.equal(g_perm, e_rt.perm)
