"""MI355X-native routed exact-token attention (HGA routed path) -- gfx950 HIP kernels behind
the reference's HierarchicalGlobalAttentionRouted / ChunkRouter interfaces."""
from ._lib import HgaError, build, lib
from .routed_attention import HierarchicalGlobalAttentionRouted, RMSNorm
from .router import (ChunkPlacementPolicy, ChunkRouter, RamKVCacheStore, RoutedKV, RouterConfig,
                     VramKVCacheStore)

__all__ = [
    "HierarchicalGlobalAttentionRouted", "RMSNorm", "ChunkPlacementPolicy", "ChunkRouter",
    "RoutedKV", "RouterConfig", "VramKVCacheStore", "RamKVCacheStore", "HgaError", "build", "lib",
]
