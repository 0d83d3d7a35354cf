"""MI355X-native mixture-of-experts feed-forward path for Garuda (hanumanit/garuda).

The hot path (routing, dispatch, packed-GGUF SwiGLU experts, combine) is hand-written
HIP for gfx950 in garuda_amd/csrc, exposed through the C-ABI in include/garuda_moe.h.
This package is the host-side mirror of the reference interface on top of it.
"""
from .moe import (  # noqa: F401
    COMBINE_EXPERT_ORDER, COMBINE_RANK_ORDER, F16, F32, GATING_DEEPSEEK, GATING_LLAMA,
    GATING_MIXTRAL, GATING_QWEN, MATH_F32, MATH_PACKED, Q2_K, Q3_K, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0,
    CacheError, ConfigError, Device, DeviceError, GarudaError, InferenceError, ModelError,
    DenseWeight, InvalidTokenError, MoeLayer, NotFoundError, block_layout, byte_size, fill_gaussian, quantize,
)
from .model import DecodeModel  # noqa: F401
from .tiers import TIER_L2, TIER_L3, TIER_SYNTHESISED, ExpertTier, engine_weights, fill_seeded  # noqa: F401
from .gguf import Gguf, TensorInfo, Value, write_gguf  # noqa: F401
