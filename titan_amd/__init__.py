"""titan_amd -- MI355X (gfx950) paged KV-cache hot path for Titan.

Drop-in for engine-kvcache's PagedKvCache and engine-cuda's PagedKvGpu /
PagedAttention / FlashAttention2 surfaces: hand-written HIP kernels compiled
offline to gfx950 code objects, launched through the C-ABI library
libengine_hip.so (include/engine_hip.h).  There is no CPU fallback.
"""
from .errors import HipError, KvCacheError
from .paged_kv import KvDataType, PagedKvGpu, PagedKvLayout
from .paged_attention import (MAX_ATTN_HEADS, MAX_FLASH_DECODING_SPLITS, MAX_HEAD_DIM,
                              PagedAttention)
from .flash_attention import FlashAttention2
from .kvcache import PagedKvCache, PagedKvCacheConfig

__all__ = [
    "HipError", "KvCacheError", "KvDataType", "PagedKvGpu", "PagedKvLayout", "PagedAttention",
    "FlashAttention2",
    "PagedKvCache", "PagedKvCacheConfig", "MAX_ATTN_HEADS", "MAX_FLASH_DECODING_SPLITS",
    "MAX_HEAD_DIM",
]
__version__ = "0.1.0"
