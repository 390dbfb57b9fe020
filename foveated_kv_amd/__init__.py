"""MI355X-native FoveatedKV decode hot path.

Two-tier KV cache (fp16 near tier, fp8-E4M3 K / INT4 V or TurboQuant far
tier) with a fused split-K decode attention kernel for gfx950, exposed
through the reference's Python tier-cache API (``MLXTierConfig``,
``MLXFoveatedLayer``, ``MLXFoveatedKVCache``, the patched attention closure)
on PyTorch-ROCm.  The HIP library ``libfkv.so`` (C ABI in include/fkv.h) is
required; nothing here falls back to a CPU path.
"""

from .tier_cache import (
    FoveatedKVCache,
    FoveatedLayer,
    MLXFoveatedKVCache,
    MLXFoveatedLayer,
    MLXTierConfig,
    TierConfig,
    standard_attention,
    standard_attention_mlx,
)
from .ext import is_available

__all__ = [
    "FoveatedKVCache",
    "FoveatedLayer",
    "TierConfig",
    "MLXFoveatedKVCache",
    "MLXFoveatedLayer",
    "MLXTierConfig",
    "standard_attention",
    "standard_attention_mlx",
    "is_available",
]
