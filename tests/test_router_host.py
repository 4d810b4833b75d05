"""Host logic of the router that runs before any kernel (CPU, no GPU needed)."""
import types

import pytest
import torch

from hierarchicalglobalattention_amd.router import (ChunkPlacementPolicy, ChunkRouter,
                                                    RouterConfig)


def test_long_fresh_block_error_names_the_limit():
    """A fresh block whose last query chunk routes over more than the chunk-parallel router's
    512 pool chunks is refused with guidance before any kernel runs (no GPU needed: the check
    precedes the first launch)."""
    pol = ChunkPlacementPolicy(keep_first=2, keep_last=8, first_token_level=True)
    router = ChunkRouter(RouterConfig(nhead=2, kv_heads=1, head_dim=16, chunk_size=8,
                                      group_size=4, topk_chunks=2, topk_groups=4, theta=1e4),
                         types.SimpleNamespace(policy=pol))
    S = (512 + 2 + 8 + 2) * 8                     # last query chunk's pool: 513 chunks
    q = torch.zeros(1, 2, S, 16)
    kv = torch.zeros(1, 1, S, 16)
    with pytest.raises(ValueError, match="512"):
        router._prefill(0, q, kv, kv, kv, None, None, populate_store=False)
