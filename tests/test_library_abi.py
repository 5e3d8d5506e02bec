"""The C-ABI library loads on the CPU and exports every entry point include/yvmoe.h declares;
host-side argument checks reject bad shapes before any GPU work (no GPU needed)."""
import ctypes
import os
import re

import pytest

from pisceslx_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "yvmoe.h")).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(yvmoe_\w+)\s*\(", text, re.M)))


def test_header_and_binding_agree():
    assert declared_functions() == sorted(_lib.EXPORTED_SYMBOLS)


def test_library_exports_every_symbol():
    l = _lib.lib()
    for name in declared_functions():
        assert hasattr(l, name), name
    assert l.yvmoe_version() == 1


def _router(E=8, k=2):
    return _lib.Router(E, 64, k, 0, 0, 4, 1.0, None, None, None, None, None)


def test_workspace_bytes_is_host_only():
    l = _lib.lib()
    r = _router(64, 6)
    e = _lib.ExpertWeights(_lib.W_INT8, 64, 2, 4096, 1408, 1, 1, 1, 1, 1, 1)
    small = l.yvmoe_workspace_bytes(64, _lib.ACT_BF16, ctypes.byref(r), ctypes.byref(e))
    big = l.yvmoe_workspace_bytes(16384, _lib.ACT_BF16, ctypes.byref(r), ctypes.byref(e))
    assert 0 < small < big
    # y [N*(k+S)][H] bf16 and h [N*(k+S)][F] bf16 dominate
    assert big >= 16384 * 8 * (4096 + 1408) * 2


@pytest.mark.parametrize("N,H,E,splits", [
    (16721, 4096, 64, 3),   # cfg3 prefill: 66 tiles x 3 splits = 198 work-groups, one round
    (8192, 7168, 256, 4),   # cfg5: 32 tiles x 2 column blocks x 4 splits = 256
    (4344, 5120, 128, 7),   # cfg4: 17 x 2 x 7 = 238 (splits of 12 k-steps, the last 8)
    (512, 4096, 64, 16),    # 2 tiles: the most splits
    (64, 4096, 64, 16),     # decode: the streaming form's 16 splits
])
def test_router_split_partials(N, H, E, splits):
    """The router GEMM's K splits, seen through the partial-sum workspace it asks for: one
    fp32 [N][Ep + 192] array per split (none without a split)."""
    r = _lib.Router(E, H, 6, 0, 0, 4, 1.0, None, None, None, None, None)
    ld = (E + 15) // 16 * 16 + 3 * _lib.PREDICTOR_DIM
    want = -(-(splits * N * ld * 4) // 256) * 256
    assert _lib.lib().yvmoe_router_workspace_bytes(N, _lib.ACT_BF16, ctypes.byref(r)) == want


@pytest.mark.parametrize("E,k,code", [(0, 1, _lib.YVMOE_ERR_SHAPE), (257, 2, _lib.YVMOE_ERR_SHAPE),
                                      (8, 9, _lib.YVMOE_ERR_SHAPE), (8, 0, _lib.YVMOE_ERR_SHAPE),
                                      (64, 17, _lib.YVMOE_ERR_SHAPE)])
def test_route_rejects_bad_shapes(E, k, code):
    l = _lib.lib()
    r = _router(E, k)
    o = _lib.Routing(1, 1, 1, 1, 1, 1, 1)
    rc = l.yvmoe_route(None, max(E, 1), None, 10, ctypes.byref(r), 4, ctypes.byref(o), None, 0, None)
    assert rc == code
    assert l.yvmoe_last_error()


def test_route_rejects_small_workspace():
    l = _lib.lib()
    r = _router(8, 2)
    o = _lib.Routing(1, 1, 1, 1, 1, 1, 1)
    rc = l.yvmoe_route(1, 8, None, 100, ctypes.byref(r), 4, ctypes.byref(o), 1, 16, None)
    assert rc == _lib.YVMOE_ERR_WORKSPACE
    with pytest.raises(ValueError, match="workspace"):
        _lib.check(rc, "yvmoe_route")


def test_forward_rejects_format_mismatch():
    l = _lib.lib()
    r = _lib.Router(8, 256, 2, 0, 1, 4, 1.0, 1, 1, 1, 1, None)
    e = _lib.ExpertWeights(_lib.W_INT8, 8, 1, 256, 512, 1, 1, 1, 1, 1, 1)
    o = _lib.Routing(1, 1, 1, 1, 1, 1, 1)
    rc = l.yvmoe_forward(1, _lib.ACT_F32, 4, ctypes.byref(r), ctypes.byref(e), 1, None, 1, 1,
                         ctypes.byref(o), 1, 1 << 30, None)
    assert rc == _lib.YVMOE_ERR_DTYPE
    e = _lib.ExpertWeights(_lib.W_INT4, 8, 1, 192, 512, 1, 1, 1, 1, 1, 1)
    rc = l.yvmoe_forward(1, _lib.ACT_BF16, 4, ctypes.byref(r), ctypes.byref(e), 1, None, 1, 1,
                         ctypes.byref(o), 1, 1 << 30, None)
    assert rc in (_lib.YVMOE_ERR_SHAPE,)


def test_python_binding_refuses_cpu_tensors():
    import torch
    from pisceslx_amd import functional as yvf
    st = yvf.RouterState(8, 64, 2, False, False, 4, 1.0, torch.zeros(1), None, None, None, None)
    with pytest.raises(ValueError, match="GPU only"):
        yvf.route(torch.zeros(4, 8), st, predictor=False, capacity_override=4)
