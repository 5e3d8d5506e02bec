"""MI355X-native (gfx950) inference forward of the Yv MoE layer.

Host side: PyTorch modules that mirror the reference interfaces (YvStableMoEGate,
YvDynamicMoELayer, YvDeepSeekMoELayer). Native side: libyvmoe.so, hand-written HIP kernels
behind the C ABI in include/yvmoe.h.
"""
from . import _lib
from .gate import YvStableMoEGate
from .layer import YvDeepSeekMoELayer, YvDynamicMoELayer
from .quant import PackedExperts, pack_experts, pack_router

__all__ = ["YvStableMoEGate", "YvDynamicMoELayer", "YvDeepSeekMoELayer", "PackedExperts",
           "pack_experts", "pack_router", "_lib"]
