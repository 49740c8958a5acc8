"""MI355X-native quantized KV-cache decode path (HIP/CDNA4).

Drop-in for the decode (q_len == 1) path of zilangchen/LLM_KVCache_Quantization:
quantize-on-append into the cache and fused quantized decode attention, behind the
reference's Python API (``decode_attn_int8``, ``decode_attn_int4``, ``INT8KVCache``,
``INT4KVCache``, ``FP16KVCache``), its attention hook (``apply_int8_fused_patch``,
``INT8CacheWrapperContainer``) and its kv_mode switch (``generate_from_ids``).  The kernels are in ``csrc/``, the C ABI is ``include/kvq.h`` and the
library is loaded through ctypes by ``_capi``.  Nothing here computes on a fallback:
without ``libkvq.so`` every kernel entry point raises.
"""
from .kernels import (  # noqa: F401
    DecodePlan,
    decode_attn_int4,
    decode_attn_int4_asym,
    decode_attn_int4_asym_gqa,
    decode_attn_int4_asym_v2,
    decode_attn_int4_kivi,
    decode_attn_int8,
    decode_attn_k8v4,
    tile_v,
    untile_v,
)
from .cache import (  # noqa: F401
    FP16KVCache,
    INT4AsymKVCache,
    INT4KVCache,
    INT8KVCache,
    K8V4KVCache,
    KIVIStyleKVCache,
    MixedKVCache,
    RoleAwareAllocatorKVCache,
    RoleAwareAsymKVCache,
    load_per_layer_bits_from_policy,
)
from .patch import (  # noqa: F401
    INT8CacheWrapper,
    INT8CacheWrapperContainer,
    apply_int8_fused_patch,
    remove_int8_fused_patch,
)
from .modes import create_kv_cache, generate_from_ids, load_calibration  # noqa: F401

__all__ = [
    "DecodePlan",
    "decode_attn_int8",
    "decode_attn_int4",
    "decode_attn_int4_asym",
    "decode_attn_k8v4",
    "tile_v",
    "untile_v",
    "INT8KVCache",
    "FP16KVCache",
    "INT4KVCache",
    "INT4AsymKVCache",
    "K8V4KVCache",
    "KIVIStyleKVCache",
    "MixedKVCache",
    "RoleAwareAsymKVCache",
    "RoleAwareAllocatorKVCache",
    "load_per_layer_bits_from_policy",
    "decode_attn_int4_kivi",
    "decode_attn_int4_asym_v2",
    "decode_attn_int4_asym_gqa",
    "INT8CacheWrapper",
    "INT8CacheWrapperContainer",
    "apply_int8_fused_patch",
    "remove_int8_fused_patch",
    "create_kv_cache",
    "generate_from_ids",
    "load_calibration",
]
