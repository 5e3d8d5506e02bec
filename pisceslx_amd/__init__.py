"""MI355X-native (gfx950) inference forward of the Yv MoE layer.

Host side: PyTorch modules that mirror the reference interfaces (YvStableMoEGate, YvMoEGate,
YvDynamicMoELayer, YvDeepSeekMoELayer, YvRMSNorm, and the MoE half of YvHybridBlock). Native side: libyvmoe.so, hand-written HIP kernels
behind the C ABI in include/yvmoe.h.
"""
from . import _lib
from .gate import YvMoEGate, YvStableMoEGate
from .layer import YvDeepSeekMoELayer, YvDynamicMoELayer
from .norms import YvHybridBlockMLP, YvRMSNorm
from .quant import PackedExperts, pack_experts, pack_router

__all__ = ["YvStableMoEGate", "YvMoEGate", "YvDynamicMoELayer", "YvDeepSeekMoELayer",
           "YvRMSNorm", "YvHybridBlockMLP", "PackedExperts", "pack_experts", "pack_router", "_lib"]
