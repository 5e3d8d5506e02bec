"""ctypes binding of libyvmoe.so, the C ABI declared in include/yvmoe.h.

The library is built in-tree (``__graft_entry__.build()`` or ``make -C pisceslx_amd/csrc``)
and loaded from this package directory. There is no fallback: if the library is missing or
fails to load, :func:`lib` raises, so a GPU run can never silently compute on another path.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libyvmoe.so")

# enums of include/yvmoe.h
YVMOE_OK = 0
YVMOE_ERR_ARG = 1
YVMOE_ERR_SHAPE = 2
YVMOE_ERR_DTYPE = 3
YVMOE_ERR_UNSUPPORTED = 4
YVMOE_ERR_LAUNCH = 5
YVMOE_ERR_WORKSPACE = 6

ACT_F32 = 0
ACT_BF16 = 1

W_F32 = 0
W_BF16 = 1
W_INT8 = 2
W_INT4 = 3
W_FP8 = 4

MAX_EXPERTS = 256
MAX_TOPK = 16
MAX_SHARED = 8
PREDICTOR_DIM = 64
STATIC_SCRATCH_BYTES = 64 << 20

EXPORTED_SYMBOLS = (
    "yvmoe_last_error",
    "yvmoe_version",
    "yvmoe_workspace_bytes",
    "yvmoe_router_workspace_bytes",
    "yvmoe_router_logits",
    "yvmoe_route",
    "yvmoe_expert_ffn",
    "yvmoe_dispatch_workspace_bytes",
    "yvmoe_dispatch",
    "yvmoe_combine",
    "yvmoe_forward",
    "yvmoe_forward_static",
    "yvmoe_moegate_workspace_bytes",
    "yvmoe_moegate_logits",
    "yvmoe_moegate_forward_workspace_bytes",
    "yvmoe_moegate_forward",
    "yvmoe_forward_moegate_workspace_bytes",
    "yvmoe_forward_moegate",
    "yvmoe_rmsnorm",
)

# YvMoEGate auxiliary heads (YVMOE_HEAD_*)
HEAD_HICL = 1
HEAD_GOT = 2
HEAD_SOFT = 4
HEAD_EO = 8


class ExpertWeights(ctypes.Structure):
    _fields_ = [
        ("format", ctypes.c_int32),
        ("num_routed", ctypes.c_int32),
        ("num_shared", ctypes.c_int32),
        ("hidden", ctypes.c_int32),
        ("ffn", ctypes.c_int32),
        ("w_gate", ctypes.c_void_p),
        ("w_up", ctypes.c_void_p),
        ("w_down", ctypes.c_void_p),
        ("s_gate", ctypes.c_void_p),
        ("s_up", ctypes.c_void_p),
        ("s_down", ctypes.c_void_p),
    ]


class Router(ctypes.Structure):
    _fields_ = [
        ("num_experts", ctypes.c_int32),
        ("hidden", ctypes.c_int32),
        ("top_k", ctypes.c_int32),
        ("fixed_shape_mode", ctypes.c_int32),
        ("dynamic_capacity", ctypes.c_int32),
        ("min_capacity", ctypes.c_int32),
        ("capacity_factor", ctypes.c_double),
        ("w_router", ctypes.c_void_p),
        ("b1", ctypes.c_void_p),
        ("w2", ctypes.c_void_p),
        ("b2", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
    ]


class Routing(ctypes.Structure):
    _fields_ = [
        ("weights", ctypes.c_void_p),
        ("indices", ctypes.c_void_p),
        ("counts", ctypes.c_void_p),
        ("offsets", ctypes.c_void_p),
        ("perm", ctypes.c_void_p),
        ("pos", ctypes.c_void_p),
        ("capacity", ctypes.c_void_p),
    ]


class RMSNormParams(ctypes.Structure):
    """yvmoe_rmsnorm_params (include/yvmoe.h)."""
    _fields_ = [
        ("weight", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("eps", ctypes.c_float),
        ("reserved", ctypes.c_int32),
    ]


class MoEGate(ctypes.Structure):
    _fields_ = [
        ("num_experts", ctypes.c_int32),
        ("hidden", ctypes.c_int32),
        ("enc_dim", ctypes.c_int32),
        ("dg_dim", ctypes.c_int32),
        ("sparsity_k", ctypes.c_int32),
        ("n_modalities", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("w_proj", ctypes.c_void_p),
        ("dg_bias", ctypes.c_void_p),
        ("prototypes_t", ctypes.c_void_p),
        ("eo_mat", ctypes.c_void_p),
        ("modal_affinity", ctypes.c_void_p),
        ("expert_bias", ctypes.c_void_p),
        ("w_hicl", ctypes.c_float),
        ("w_got", ctypes.c_float),
        ("w_soft", ctypes.c_float),
        ("w_eo", ctypes.c_float),
        ("soft_temperature", ctypes.c_float),
        ("temperature", ctypes.c_float),
        ("soft_eps", ctypes.c_float),
        ("load_balance_alpha", ctypes.c_float),
        ("z_loss_alpha", ctypes.c_float),
        ("soft_budget", ctypes.c_float),
        ("capacity_loss", ctypes.c_float),
        ("reserved_f", ctypes.c_float),
    ]


_LIB: Optional[ctypes.CDLL] = None


def _declare(l: ctypes.CDLL) -> None:
    vp, i32, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_size_t
    l.yvmoe_last_error.restype = ctypes.c_char_p
    l.yvmoe_last_error.argtypes = []
    l.yvmoe_version.restype = i32
    l.yvmoe_version.argtypes = []
    l.yvmoe_workspace_bytes.restype = sz
    l.yvmoe_workspace_bytes.argtypes = [i32, i32, ctypes.POINTER(Router), ctypes.POINTER(ExpertWeights)]
    l.yvmoe_router_workspace_bytes.restype = sz
    l.yvmoe_router_workspace_bytes.argtypes = [i32, i32, ctypes.POINTER(Router)]
    l.yvmoe_router_logits.restype = i32
    l.yvmoe_router_logits.argtypes = [vp, i32, i32, ctypes.POINTER(Router), vp, i32, vp, sz, vp]
    l.yvmoe_route.restype = i32
    l.yvmoe_route.argtypes = [vp, i32, vp, i32, ctypes.POINTER(Router), i32,
                              ctypes.POINTER(Routing), vp, sz, vp]
    l.yvmoe_expert_ffn.restype = i32
    l.yvmoe_expert_ffn.argtypes = [vp, i32, i32, i32, ctypes.POINTER(ExpertWeights),
                                   ctypes.POINTER(Routing), vp, vp, sz, vp]
    l.yvmoe_dispatch_workspace_bytes.restype = sz
    l.yvmoe_dispatch_workspace_bytes.argtypes = [i32, i32, i32, ctypes.POINTER(ExpertWeights)]
    l.yvmoe_dispatch.restype = i32
    l.yvmoe_dispatch.argtypes = [vp, i32, i32, vp, i32, vp, i32, ctypes.POINTER(ExpertWeights),
                                 vp, vp, vp, vp, vp, vp, sz, vp]
    l.yvmoe_combine.restype = i32
    l.yvmoe_combine.argtypes = [vp, i32, i32, i32, i32, i32, ctypes.POINTER(Routing), vp, vp,
                                vp, vp, vp]
    l.yvmoe_moegate_workspace_bytes.restype = sz
    l.yvmoe_moegate_workspace_bytes.argtypes = [i32, i32, ctypes.POINTER(MoEGate)]
    l.yvmoe_moegate_logits.restype = i32
    l.yvmoe_moegate_logits.argtypes = [vp, i32, i32, ctypes.POINTER(MoEGate), vp, vp, vp, vp, sz, vp]
    l.yvmoe_moegate_forward_workspace_bytes.restype = sz
    l.yvmoe_moegate_forward_workspace_bytes.argtypes = [i32, i32, i32, ctypes.POINTER(MoEGate)]
    l.yvmoe_moegate_forward.restype = i32
    l.yvmoe_moegate_forward.argtypes = [vp, i32, i32, ctypes.POINTER(MoEGate), vp, i32, vp, vp,
                                        ctypes.POINTER(Routing), vp, sz, vp]
    l.yvmoe_forward_moegate_workspace_bytes.restype = sz
    l.yvmoe_forward_moegate_workspace_bytes.argtypes = [i32, i32, i32, ctypes.POINTER(MoEGate),
                                                        ctypes.POINTER(ExpertWeights)]
    l.yvmoe_forward_moegate.restype = i32
    l.yvmoe_forward_moegate.argtypes = [vp, i32, i32, ctypes.POINTER(MoEGate), vp, i32, vp,
                                        ctypes.POINTER(ExpertWeights), vp, vp, vp, vp,
                                        ctypes.POINTER(Routing), vp, vp, vp, sz, vp]
    l.yvmoe_rmsnorm.restype = i32
    l.yvmoe_rmsnorm.argtypes = [vp, i32, i32, i32, ctypes.POINTER(RMSNormParams), i32, vp, vp]
    l.yvmoe_forward_static.restype = i32
    l.yvmoe_forward_static.argtypes = [vp, i32, i32, ctypes.POINTER(Router),
                                       ctypes.POINTER(ExpertWeights), vp, vp, vp, vp,
                                       ctypes.POINTER(Routing), vp]
    l.yvmoe_forward.restype = i32
    l.yvmoe_forward.argtypes = [vp, i32, i32, ctypes.POINTER(Router), ctypes.POINTER(ExpertWeights),
                                vp, vp, vp, vp, ctypes.POINTER(Routing), vp, sz, vp]


def lib() -> ctypes.CDLL:
    """Load libyvmoe.so from the package directory (raises if it is not built)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built: run `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `make -C pisceslx_amd/csrc`")
        l = ctypes.CDLL(LIB_PATH)
        _declare(l)
        _LIB = l
    return _LIB


def check(rc: int, what: str) -> None:
    """Raise the Python exception that matches a yvmoe_status."""
    if rc == YVMOE_OK:
        return
    msg = lib().yvmoe_last_error().decode(errors="replace")
    text = f"{what}: {msg} (status {rc})"
    if rc in (YVMOE_ERR_ARG, YVMOE_ERR_SHAPE, YVMOE_ERR_DTYPE, YVMOE_ERR_WORKSPACE):
        raise ValueError(text)
    if rc == YVMOE_ERR_UNSUPPORTED:
        raise NotImplementedError(text)
    raise RuntimeError(text)
