"""Host logic of the router that runs before any kernel (CPU, no GPU needed)."""
import types

import pytest
import torch

from hierarchicalglobalattention_amd.router import (ChunkPlacementPolicy, ChunkRouter,
                                                    RouterConfig)


@pytest.mark.parametrize("dtype,head_dim,limit", [(torch.float32, 16, 512),
                                                   (torch.bfloat16, 64, 2048)])
def test_long_fresh_block_error_names_the_limit(dtype, head_dim, limit):
    """A fresh block whose last query chunk routes over more chunks than the chunk-parallel
    router takes (512 for the split kernels and fp32; 2048 for the fused bf16 router) is refused
    with guidance before any kernel runs (no GPU needed: the check precedes the first launch).
    Blocks within the bound are routed on the GPU (tests/test_gpu_long_prefill.py)."""
    pol = ChunkPlacementPolicy(keep_first=2, keep_last=8, first_token_level=True)
    router = ChunkRouter(RouterConfig(nhead=2, kv_heads=1, head_dim=head_dim, chunk_size=8,
                                      group_size=4, topk_chunks=2, topk_groups=4, theta=1e4),
                         types.SimpleNamespace(policy=pol))
    S = (limit + 2 + 8 + 2) * 8                   # last query chunk's pool: limit + 1 chunks
    q = torch.zeros(1, 2, S, head_dim, dtype=dtype)
    kv = torch.zeros(1, 1, S, head_dim, dtype=dtype)
    with pytest.raises(ValueError, match=str(limit)):
        router._prefill(0, q, kv, kv, kv, None, None, populate_store=False)


def test_router_requires_token_level_first_window():
    """The exact-token router attends the first window's tokens; a policy asking for a
    summary-level first window (the summary-attending variant) is refused."""
    pol = ChunkPlacementPolicy(keep_first=1, keep_last=2, first_token_level=False)
    with pytest.raises(ValueError, match="first_token_level"):
        ChunkRouter(RouterConfig(nhead=2, kv_heads=1, head_dim=16, chunk_size=8, group_size=4),
                    types.SimpleNamespace(policy=pol))


def test_routed_kv_attend_defaults_to_summaries_like_the_reference():
    """RoutedKV.attend(q, use_summaries=True) as in chunk_router.py:139; this router builds no
    summary keys, so the flag selects nothing extra."""
    import inspect

    from hierarchicalglobalattention_amd.router import RoutedKV
    assert inspect.signature(RoutedKV.attend).parameters["use_summaries"].default is True
    assert RoutedKV.summary_k is None and RoutedKV.summary_v is None


@pytest.mark.parametrize("loc,cls", [("vram", "VramKVCacheStore"), ("ram", "RamKVCacheStore"),
                                     ("fs", "FsKVCacheStore"), ("disk", "RamKVCacheStore")])
def test_unknown_cache_location_takes_the_ram_tier(loc, cls):
    """HierarchicalGlobalAttentionRouted._make_store (HierarchicalGlobalAttentionRouted.py:
    223-240): "vram" -> VRAM store, any other location -> the RAM store ("fs" is this
    package's on-disk tier)."""
    from hierarchicalglobalattention_amd.routed_attention import HierarchicalGlobalAttentionRouted
    m = HierarchicalGlobalAttentionRouted(d_model=32, nhead=2, kv_heads=1, cache_location=loc)
    store = m._make_store(1, torch.float32, torch.device("cpu"))
    assert type(store).__name__ == cls
    if cls == "FsKVCacheStore":
        store.close()
