"""MI355X-native routed exact-token attention (HGA routed path) -- gfx950 HIP kernels behind
the reference's HierarchicalGlobalAttentionRouted / ChunkRouter interfaces."""
from ._lib import HgaError, build, lib
from .routed_attention import HierarchicalGlobalAttentionRouted, RMSNorm
from .qwen_routed_attention import (QwenRoutedAttention, replace_qwen_attention_with_router,
                                    restore_original_attention)
from .router import (ChunkPlacementPolicy, ChunkRouter, FsKVCacheStore, RamKVCacheStore,
                     RoutedKV, RouterConfig, VramKVCacheStore)

__all__ = [
    "HierarchicalGlobalAttentionRouted", "RMSNorm", "ChunkPlacementPolicy", "ChunkRouter",
    "RoutedKV", "RouterConfig", "VramKVCacheStore", "RamKVCacheStore", "FsKVCacheStore",
    "HgaError", "build", "lib",
    "QwenRoutedAttention", "replace_qwen_attention_with_router", "restore_original_attention",
]
